"""Test fixtures rebuilt from the reference's own test data constructions.

`Fixture` follows test_attention.mojo:169-246: LCG-filled Q/K/V (:27-42), a shuffled
block table (i*37 + 11) % 160 over 160 blocks of 16 tokens (:45-50), K scaled by
`k_scale`. Planting follows :324-365 / :440-497.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

BLOCK_SIZE = 16
NUM_BLOCKS = 160
CAPACITY = NUM_BLOCKS * BLOCK_SIZE


class Fixture:
    def __init__(self, heads, kv_heads, head_dim, seed, k_scale):
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.kv_stride = kv_heads * head_dim
        rng = O.Lcg(seed)
        self.q = rng.fill(heads * head_dim, 1.0)
        self.k_pool = rng.fill(CAPACITY * self.kv_stride, k_scale)
        self.v_pool = rng.fill(CAPACITY * self.kv_stride, 1.0)
        self.table = O.shuffled_block_table(NUM_BLOCKS, NUM_BLOCKS)

    def row_of(self, t):
        return (int(self.table[t // BLOCK_SIZE]) * BLOCK_SIZE + t % BLOCK_SIZE) * self.kv_stride

    def plant(self, t):
        """Key at t aligned with every query head (x4), value 1000 (test_attention.mojo:452-460)."""
        r = self.row_of(t)
        ratio = self.heads // self.kv_heads
        for g in range(self.kv_heads):
            self.k_pool[r + g * self.head_dim: r + (g + 1) * self.head_dim] = 0.0
            self.v_pool[r + g * self.head_dim: r + (g + 1) * self.head_dim] = 1000.0
        for h in range(self.heads):
            g = h // ratio
            sl = slice(r + g * self.head_dim, r + (g + 1) * self.head_dim)
            self.k_pool[sl] += self.q[h * self.head_dim:(h + 1) * self.head_dim] * np.float32(4.0)

    def run_new(self, pos, window, nthreads=1):
        return O.paged_attention_layer(self.q, self.k_pool, self.v_pool, self.table, BLOCK_SIZE,
                                       pos, self.heads, self.kv_heads, self.head_dim, window,
                                       nthreads=nthreads)

    def run_legacy(self, pos):
        return O.legacy_paged_attention(self.q, self.k_pool, self.v_pool, self.table, BLOCK_SIZE,
                                        pos, self.heads, self.kv_heads, self.head_dim)

    def run_reference(self, pos, start_t):
        return O.attention_f64(self.q, self.k_pool, self.v_pool, self.table, BLOCK_SIZE, pos,
                               start_t, self.heads, self.kv_heads, self.head_dim)
