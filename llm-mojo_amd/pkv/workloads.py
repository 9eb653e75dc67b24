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
                 steps: int = 64, hkv: int | None = None, d: int | None = None,
                 windows: tuple | None = None, scale: float | None = None):
        self.seed = seed
        self.B = batch
        self.STEPS = steps
        if hkv is not None:
            self.HKV = hkv
        if d is not None:
            self.D = d
        # one entry per layer: its window (0 = global); the same block table serves all
        self.windows = tuple(windows) if windows is not None else (self.WINDOW, 0)
        self.L = len(self.windows)
        if scale is not None:
            self.SCALE = scale
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
        self.seed_pool = [[base + 10 * layer + kv for kv in range(2)] for layer in range(self.L)]
        self.seed_q = base + 100
        self.seed_knew, self.seed_vnew = base + 101, base + 102
        self.seed_admit_k, self.seed_admit_v = base + 103, base + 104

    @classmethod
    def engine_global(cls, seed: int = 0, **kw) -> "DecodeSchedule":
        """Config 2's schedule on the engine's own global-layer geometry: 16 q / 2 kv heads,
        head_dim 512 (model_speculative_moe_batched.mojo:1905-1907; the MTP assistant's
        last layer reads that pool too, :756-760), one full-attention layer, fp32 pools.
        Softmax scale 2^-4, as config 2 (the engine's RMS-normed Q and K take scale 1; N(0, 1)
        data needs a scale near 1/sqrt(D) to keep the softmax from collapsing onto one key,
        and a power of two keeps the scaled query exact in fp32 for the reference path,
        which multiplies q by the scale in fp32)."""
        return cls(seed=seed, hkv=2, d=512, windows=(0,), scale=0.0625, **kw)

    @property
    def admit_rows(self) -> int:
        return self.RETIRE_N * self.ADMIT_CTX

    def device_data(self, stream=None) -> dict:
        """All float inputs on the device, generated from their seeds."""
        rows = self.num_blocks * self.BS
        L = self.L
        d = {"pools": [[synth.normal((rows, self.kv_stride), self.seed_pool[l][kv],
                                     stream=stream) for kv in range(2)] for l in range(L)],
             "q": synth.normal((self.STEPS, L, self.B, 1, self.HQ, self.D), self.seed_q,
                               stream=stream),
             "k_new": synth.normal((self.STEPS, L, self.B, self.kv_stride), self.seed_knew,
                                   stream=stream),
             "v_new": synth.normal((self.STEPS, L, self.B, self.kv_stride), self.seed_vnew,
                                   stream=stream)}
        ne = max(len(self.events), 1)
        d["admit_k"] = synth.normal((ne, L, self.admit_rows, self.kv_stride),
                                    self.seed_admit_k, stream=stream)
        d["admit_v"] = synth.normal((ne, L, self.admit_rows, self.kv_stride),
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
        """Keys each sequence's query attends at step j (the layer's window, 0 = all)."""
        n = self.pos[j].astype(np.int64) + 1
        w = self.windows[layer]
        return np.minimum(n, w) if w > 0 else n

    def attend_bytes(self, j: int, layer: int, elt: int = 4) -> int:
        """Algorithmic HBM bytes of one attention launch: each attended K and V row
        slice of the kv heads once, Q in, O out, and the block-table entries read."""
        n = self.keys_attended(j, layer)
        lo = self.pos[j].astype(np.int64) + 1 - n
        pages = self.pos[j].astype(np.int64) // self.BS - lo // self.BS + 1
        kv = int(n.sum()) * 2 * self.kv_stride * elt
        qo = 2 * self.B * self.HQ * self.D * 4
        return kv + qo + int(pages.sum()) * 4


def _assign_tables(rng, blocks_per_seq, num_blocks: int, table_stride: int):
    """Seeded random non-overlapping block tables: a permutation of the pool dealt out to
    the sequences in order; the unassigned ids form the free list in ascending order (a
    fresh BlockManager's LIFO stack after the assigned ids were taken)."""
    perm = rng.permutation(num_blocks).astype(np.int32)
    B = len(blocks_per_seq)
    tables = np.zeros((B, table_stride), np.int32)
    lens = np.asarray(blocks_per_seq, np.int32)
    off = 0
    for s in range(B):
        n = int(lens[s])
        tables[s, :n] = perm[off:off + n]
        off += n
    return tables, lens, np.sort(perm[off:]).astype(np.int32)


class SingleStep:
    """Config 1: one sequence, 16 q / 8 kv heads, head_dim 256,
    block 16, fp32; a 256-block pool; the sequence holds 512 tokens in a seeded random
    32-block prefix of a permutation of the pool; the step appends the token at position
    512 (the 33rd block, popped from the back of the free list) and attends 513 keys.
    K, V, Q ~ N(0, 1); softmax scale 1/sqrt(256)."""

    HQ, HKV, D, BS = 16, 8, 256, 16
    NUM_BLOCKS = 256
    CTX = 512
    SCALE = 0.0625
    B = 1
    WINDOW = 0

    def __init__(self, seed: int = 0):
        rng = np.random.default_rng(seed)
        self.kv_stride = self.HKV * self.D
        self.num_blocks = self.NUM_BLOCKS
        self.table_stride = 64
        self.tables0, self.lens0, self.free0 = _assign_tables(
            rng, [self.CTX // self.BS], self.num_blocks, self.table_stride)
        self.pos = np.array([self.CTX], np.int32)
        self.max_pos = self.CTX
        base = int(rng.integers(1, 2**40))
        self.seed_k, self.seed_v = base, base + 1
        self.seed_q, self.seed_knew, self.seed_vnew = base + 2, base + 3, base + 4

    def device_data(self, stream=None) -> dict:
        rows = self.num_blocks * self.BS
        return {"k": synth.normal((rows, self.kv_stride), self.seed_k, stream=stream),
                "v": synth.normal((rows, self.kv_stride), self.seed_v, stream=stream),
                "q": synth.normal((1, 1, self.HQ, self.D), self.seed_q, stream=stream),
                "k_new": synth.normal((1, self.kv_stride), self.seed_knew, stream=stream),
                "v_new": synth.normal((1, self.kv_stride), self.seed_vnew, stream=stream)}

    def attend_bytes(self, elt: int = 4) -> int:
        n = self.CTX + 1
        return n * 2 * self.kv_stride * elt + 2 * self.HQ * self.D * 4 + (n // self.BS + 1) * 4


class LongDecode:
    """Config 3: batch 8, 16 q / 8 kv heads, head_dim 256,
    block 16, bf16 K/V pages, fp32 Q. A pool of exactly 16384 blocks dealt out by a seeded
    permutation, 2048 blocks (32768 slots) per sequence. Each sequence holds 32767 cached
    tokens; the step appends the token at position 32767 (the last slot of its partially
    filled 2048th block) and attends all 32768 keys. K, V ~ N(0, 1) rounded to bf16
    (round-to-nearest-even), Q ~ N(0, 1) fp32, scale 1/sqrt(256)."""

    HQ, HKV, D, BS = 16, 8, 256, 16
    B = 8
    CTX = 32768  # keys attended, including the appended token
    NUM_BLOCKS = 16384
    SCALE = 0.0625
    WINDOW = 0

    def __init__(self, seed: int = 0, batch: int | None = None, ctx: int | None = None):
        rng = np.random.default_rng(seed)
        if batch is not None:
            self.B = batch
        if ctx is not None:
            self.CTX = ctx
        self.kv_stride = self.HKV * self.D
        per_seq = (self.CTX + self.BS - 1) // self.BS
        self.num_blocks = self.NUM_BLOCKS if (batch, ctx) == (None, None) else self.B * per_seq
        self.table_stride = per_seq
        self.tables0, self.lens0, self.free0 = _assign_tables(
            rng, [per_seq] * self.B, self.num_blocks, self.table_stride)
        self.pos = np.full(self.B, self.CTX - 1, np.int32)
        self.max_pos = self.CTX - 1
        base = int(rng.integers(1, 2**40))
        self.seed_k, self.seed_v = base, base + 1
        self.seed_q, self.seed_knew, self.seed_vnew = base + 2, base + 3, base + 4

    def device_data(self, stream=None) -> dict:
        rows = self.num_blocks * self.BS
        bf = np.uint16
        return {"k": synth.normal((rows, self.kv_stride), self.seed_k, bf, stream=stream),
                "v": synth.normal((rows, self.kv_stride), self.seed_v, bf, stream=stream),
                "q": synth.normal((self.B, 1, self.HQ, self.D), self.seed_q, stream=stream),
                "k_new": synth.normal((self.B, self.kv_stride), self.seed_knew, bf,
                                      stream=stream),
                "v_new": synth.normal((self.B, self.kv_stride), self.seed_vnew, bf,
                                      stream=stream)}

    def attend_bytes(self, elt: int = 2) -> int:
        n = self.CTX
        return (self.B * n * 2 * self.kv_stride * elt + 2 * self.B * self.HQ * self.D * 4
                + self.B * ((n - 1) // self.BS + 1) * 4)


class VerifySchedule:
    """Config 5: MTP speculative verify and rollback with shared
    KV. 16 sequences with contexts seeded uniform on [512, 4096]; two global-attention
    layers (16 q / 8 kv heads, head_dim 256, fp32, block 16) standing in for the target
    layers whose pools the MTP assistant reads. Per iteration, with L = each sequence's
    committed length:
      1. MTP drafting: DRAFT read-only attention calls on both pools at kv_pos = L - 1,
         through the target's own tables (mtp_generate_step, …batched.mojo:2955-2990);
      2. verify: append DRAFT draft tokens' K/V at L .. L + DRAFT - 1 on both layers, then
         attend DRAFT query tokens against the paged prefix plus the causal-masked draft;
      3. acceptance: a seeded count a ~ U{0..DRAFT}; rollback to L + a (tail blocks back to
         the LIFO free list in ascending logical order).
    32 iterations. The pool holds the blocks the contexts can grow to, plus 10 %."""

    HQ, HKV, D, BS = 16, 8, 256, 16
    B = 16
    DRAFT = 4
    ITERS = 32
    SCALE = 0.0625
    WINDOW = 0
    LAYERS = 2

    def __init__(self, seed: int = 0, batch: int | None = None, iters: int | None = None,
                 ctx_lo: int = 512, ctx_hi: int = 4096, bf16: bool = False):
        rng = np.random.default_rng(seed)
        self.bf16 = bf16  # bf16 pools and appended rows (the bf16 variant); fp32 by default
        self.elt = 2 if bf16 else 4
        if batch is not None:
            self.B = batch
        if iters is not None:
            self.ITERS = iters
        B, bs = self.B, self.BS
        self.kv_stride = self.HKV * self.D
        self.ctx0 = rng.integers(ctx_lo, ctx_hi + 1, B).astype(np.int64)
        grow = self.DRAFT * (self.ITERS + 1)
        need = int(np.sum((self.ctx0 + grow + bs - 1) // bs))
        self.num_blocks = int(np.ceil(need * 1.1))
        self.table_stride = int((ctx_hi + grow + bs - 1) // bs) + 2
        self.tables0, self.lens0, self.free0 = _assign_tables(
            rng, (self.ctx0 + bs - 1) // bs, self.num_blocks, self.table_stride)
        self.accept = rng.integers(0, self.DRAFT + 1, (self.ITERS, B)).astype(np.int32)
        self.length = np.zeros((self.ITERS + 1, B), np.int64)  # committed length per iter
        self.length[0] = self.ctx0
        for it in range(self.ITERS):
            self.length[it + 1] = self.length[it] + self.accept[it]
        self.max_pos = int(self.length.max()) + self.DRAFT - 1
        base = int(rng.integers(1, 2**40))
        self.seed_pool = [[base + 10 * layer + kv for kv in range(2)] for layer in range(2)]
        self.seed_q, self.seed_mtp_q = base + 100, base + 101
        self.seed_knew, self.seed_vnew = base + 102, base + 103

    def device_data(self, stream=None) -> dict:
        rows = self.num_blocks * self.BS
        n = self.ITERS * self.LAYERS
        kv = np.uint16 if self.bf16 else np.float32
        return {"pools": [[synth.normal((rows, self.kv_stride), self.seed_pool[l][i], kv,
                                        stream=stream) for i in range(2)]
                          for l in range(self.LAYERS)],
                "q": synth.normal((n, self.B, self.DRAFT, self.HQ, self.D), self.seed_q,
                                  stream=stream),
                "mtp_q": synth.normal((n, self.DRAFT, self.B, 1, self.HQ, self.D),
                                      self.seed_mtp_q, stream=stream),
                "k_new": synth.normal((n, self.B * self.DRAFT, self.kv_stride), self.seed_knew,
                                      kv, stream=stream),
                "v_new": synth.normal((n, self.B * self.DRAFT, self.kv_stride), self.seed_vnew,
                                      kv, stream=stream)}

    def pos(self, it: int) -> np.ndarray:
        return self.length[it].astype(np.int32)

    def new_len(self, it: int) -> np.ndarray:
        return self.length[it + 1].astype(np.int32)

    def tok_off(self) -> np.ndarray:
        return (np.arange(self.B + 1) * self.DRAFT).astype(np.int32)

    def verify_bytes(self, it: int, elt: int | None = None) -> int:
        """Algorithmic bytes of one verify attention launch (one layer): each K/V row
        slice of prefix + draft once, Q in, O out, table entries."""
        elt = self.elt if elt is None else elt
        n = self.length[it] + self.DRAFT
        kv = int(n.sum()) * 2 * self.kv_stride * elt
        qo = 2 * self.B * self.DRAFT * self.HQ * self.D * 4
        return kv + qo + int(((n - 1) // self.BS + 1).sum()) * 4

    def verify_flops(self, it: int) -> int:
        """QK^T and PV multiply-adds x 2 of one verify launch, counting the causal mask:
        query j attends L + j + 1 keys."""
        keys = sum(int(self.length[it, s]) * self.DRAFT
                   + self.DRAFT * (self.DRAFT + 1) // 2 for s in range(self.B))
        return 4 * self.D * self.HQ * keys


class PrefillChunk:
    """Config 4: chunked prefill into the paged cache, bf16,
    MFMA path. 4 sequences, 16 q / 8 kv heads, head_dim 256, block 16. Each sequence
    already holds a prefix of seeded length in [0, 6144] (seeded random block tables);
    a 2048-token chunk of Q/K/V ~ N(0, 1) bf16 is appended (the chunk fills the prefix's
    partial last block, then freshly allocated blocks popped from the LIFO free list) and
    every chunk query attends causally over prefix plus chunk, fp32 accumulation. The pool
    holds the blocks prefix + chunk need, plus 10 %."""

    HQ, HKV, D, BS = 16, 8, 256, 16
    B = 4
    CHUNK = 2048
    PREFIX_MAX = 6144
    SCALE = 0.0625
    WINDOW = 0

    def __init__(self, seed: int = 0, batch: int | None = None, chunk: int | None = None,
                 prefix_max: int | None = None, hq: int | None = None, hkv: int | None = None,
                 window: int | None = None, prefix=None):
        rng = np.random.default_rng(seed)
        for name, v in (("B", batch), ("CHUNK", chunk), ("PREFIX_MAX", prefix_max),
                        ("HQ", hq), ("HKV", hkv), ("WINDOW", window)):
            if v is not None:
                setattr(self, name, v)
        B, bs = self.B, self.BS
        self.kv_stride = self.HKV * self.D
        self.prefix = rng.integers(0, self.PREFIX_MAX + 1, B).astype(np.int64)
        if prefix is not None:
            self.prefix = np.asarray(prefix, np.int64)
        need = int(np.sum((self.prefix + self.CHUNK + bs - 1) // bs))
        self.num_blocks = int(np.ceil(need * 1.1))
        self.table_stride = int((self.PREFIX_MAX + self.CHUNK + bs - 1) // bs) + 2
        self.tables0, self.lens0, self.free0 = _assign_tables(
            rng, (self.prefix + bs - 1) // bs, self.num_blocks, self.table_stride)
        self.pos = self.prefix.astype(np.int32)
        self.max_pos = int(self.prefix.max()) + self.CHUNK - 1
        base = int(rng.integers(1, 2**40))
        self.seed_k, self.seed_v = base, base + 1
        self.seed_q, self.seed_knew, self.seed_vnew = base + 2, base + 3, base + 4

    @property
    def rows(self) -> int:
        return self.B * self.CHUNK

    def tok_off(self) -> np.ndarray:
        return (np.arange(self.B + 1) * self.CHUNK).astype(np.int32)

    def device_data(self, stream=None) -> dict:
        bf = np.uint16
        prow = self.num_blocks * self.BS
        return {"k": synth.normal((prow, self.kv_stride), self.seed_k, bf, stream=stream),
                "v": synth.normal((prow, self.kv_stride), self.seed_v, bf, stream=stream),
                "q": synth.normal((self.rows, self.HQ, self.D), self.seed_q, bf, stream=stream),
                "k_new": synth.normal((self.rows, self.kv_stride), self.seed_knew, bf,
                                      stream=stream),
                "v_new": synth.normal((self.rows, self.kv_stride), self.seed_vnew, bf,
                                      stream=stream)}

    def keys_attended(self) -> int:
        """Sum over all queries of the keys each attends (causal, window 0 or W)."""
        tot = 0
        for s in range(self.B):
            p = np.arange(self.CHUNK, dtype=np.int64) + int(self.prefix[s])
            lo = np.maximum(p - self.WINDOW + 1, 0) if self.WINDOW > 0 else np.zeros_like(p)
            tot += int((p - lo + 1).sum())
        return tot

    def flops(self) -> int:
        """QK^T and PV: 2 multiply-adds per (query, head, key, dim) -> 4 flops."""
        return 4 * self.D * self.HQ * self.keys_attended()

    def kv_bytes(self, elt: int = 2) -> int:
        """K and V of every sequence's prefix + chunk read once per kv head."""
        return int((self.prefix + self.CHUNK).sum()) * 2 * self.kv_stride * elt
