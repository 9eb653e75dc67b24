"""Seeded synthetic workloads for the benchmark configurations.

Config 2 (the headline): continuous-batching decode of B=32 sequences on one sliding
(window 1024) and one global layer, 16 query / 8 KV heads, head_dim 256, block 16, fp32.
Contexts uniform on [128, 8192]; the pool holds the blocks needed for the contexts plus
the decode steps, plus 10 % free; block tables are a seeded random non-overlapping
assignment and the free list holds the unassigned ids in ascending order. Each step
appends one token per sequence to both layers and attends; every 8 steps 4 seeded
sequences retire (their blocks return to the free list, ascending) and 4 new sequences
with 256-token contexts are admitted into the freed slots. K, V and Q ~ N(0, 1); the
softmax scale is 1/sqrt(256) = 2^-4.

Integer structure (contexts, tables, events) is drawn on the host with numpy; float data
comes from device-side seeded normal streams (pkv.synth), each identified by a seed.
"""
from __future__ import annotations

import numpy as np

from . import hip, synth


class DecodeSchedule:
    """Config 2: initial tables / free list, every step's
    positions and admissions, and the seeds of all float data."""

    HQ, HKV, D = 16, 8, 256
    BS = 16
    WINDOW = 1024
    RETIRE_EVERY = 8
    RETIRE_N = 4
    ADMIT_CTX = 256
    SCALE = 0.0625

    def __init__(self, seed: int = 0, batch: int = 32, ctx_lo: int = 128, ctx_hi: int = 8192,
                 steps: int = 64):
        self.seed = seed
        self.B = batch
        self.STEPS = steps
        rng = np.random.default_rng(seed)
        B, bs = self.B, self.BS
        self.kv_stride = self.HKV * self.D
        self.ctx0 = rng.integers(ctx_lo, ctx_hi + 1, B).astype(np.int64)
        need = int(np.sum((self.ctx0 + steps + bs - 1) // bs))
        self.num_blocks = int(np.ceil(need * 1.1))
        perm = rng.permutation(self.num_blocks).astype(np.int32)
        nblk = (self.ctx0 + bs - 1) // bs
        self.table_stride = int((ctx_hi + steps + bs - 1) // bs) + 2
        self.tables0 = np.zeros((B, self.table_stride), np.int32)
        self.lens0 = nblk.astype(np.int32)
        off = 0
        for s in range(B):
            self.tables0[s, :nblk[s]] = perm[off:off + nblk[s]]
            off += int(nblk[s])
        self.free0 = np.sort(perm[off:]).astype(np.int32)
        length = self.ctx0.copy()
        self.events = {}  # step -> retired slots (ascending); admitted into the same slots
        self.pos = np.zeros((steps, B), np.int32)
        for j in range(steps):
            if j > 0 and j % self.RETIRE_EVERY == 0:
                slots = np.sort(rng.choice(B, self.RETIRE_N, replace=False)).astype(np.int32)
                self.events[j] = slots
                length[slots] = self.ADMIT_CTX
            self.pos[j] = length.astype(np.int32)
            length += 1
        self.max_pos = int(self.pos.max())
        base = int(rng.integers(1, 2**40))
        # seeds of the float streams
        self.seed_pool = [[base + 10 * layer + kv for kv in range(2)] for layer in range(2)]
        self.seed_q = base + 100
        self.seed_knew, self.seed_vnew = base + 101, base + 102
        self.seed_admit_k, self.seed_admit_v = base + 103, base + 104

    @property
    def admit_rows(self) -> int:
        return self.RETIRE_N * self.ADMIT_CTX

    def device_data(self, stream=None) -> dict:
        """All float inputs on the device, generated from their seeds."""
        rows = self.num_blocks * self.BS
        d = {"pools": [[synth.normal((rows, self.kv_stride), self.seed_pool[l][kv],
                                     stream=stream) for kv in range(2)] for l in range(2)],
             "q": synth.normal((self.STEPS, 2, self.B, 1, self.HQ, self.D), self.seed_q,
                               stream=stream),
             "k_new": synth.normal((self.STEPS, 2, self.B, self.kv_stride), self.seed_knew,
                                   stream=stream),
             "v_new": synth.normal((self.STEPS, 2, self.B, self.kv_stride), self.seed_vnew,
                                   stream=stream)}
        ne = max(len(self.events), 1)
        d["admit_k"] = synth.normal((ne, 2, self.admit_rows, self.kv_stride),
                                    self.seed_admit_k, stream=stream)
        d["admit_v"] = synth.normal((ne, 2, self.admit_rows, self.kv_stride),
                                    self.seed_admit_v, stream=stream)
        d["event_index"] = {j: i for i, j in enumerate(sorted(self.events))}
        return d

    # ---- per-event arrays
    def retire_new_len(self, j: int) -> np.ndarray:
        nl = np.full(self.B, -1, np.int32)
        nl[self.events[j]] = 0
        return nl

    def admit_pos(self, j: int) -> np.ndarray:
        p = np.full(self.B, -1, np.int32)
        p[self.events[j]] = 0
        return p

    def admit_tok_off(self, j: int) -> np.ndarray:
        n = np.zeros(self.B, np.int64)
        n[self.events[j]] = self.ADMIT_CTX
        return np.concatenate([[0], np.cumsum(n)]).astype(np.int32)

    def decode_tok_off(self) -> np.ndarray:
        return np.arange(self.B + 1, dtype=np.int32)

    def keys_attended(self, j: int, layer: int) -> np.ndarray:
        """Keys each sequence's query attends at step j (window 1024 on layer 0)."""
        n = self.pos[j].astype(np.int64) + 1
        return np.minimum(n, self.WINDOW) if layer == 0 else n

    def attend_bytes(self, j: int, layer: int, elt: int = 4) -> int:
        """Algorithmic HBM bytes of one attention launch: each attended K and V row
        slice of the kv heads once, Q in, O out, and the block-table entries read."""
        n = self.keys_attended(j, layer)
        lo = self.pos[j].astype(np.int64) + 1 - n
        pages = self.pos[j].astype(np.int64) // self.BS - lo // self.BS + 1
        kv = int(n.sum()) * 2 * self.kv_stride * elt
        qo = 2 * self.B * self.HQ * self.D * 4
        return kv + qo + int(pages.sum()) * 4
