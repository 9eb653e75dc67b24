"""CPU checks that pin the oracle's block bookkeeping (BlockManager, append, rollback).

The reference has no tests for these (they live in the engine's main scope); they are
pinned here by (a) a literal Python transcription of the engine's per-token code on
Python lists, run on random op sequences, and (b) invariants: every block is in exactly
one table or in the free list, LIFO order, rows hold exact copies, and rollback then
re-append reproduces a fresh run from the same free-list state.
"""
import numpy as np
import pytest

from oracle import oracle as O


def test_block_manager_lifo():
    # …batched.mojo:789-807: init [0..max-1]; allocate pops the back; free pushes back.
    bm = O.BlockManager(4)
    assert list(bm.free_blocks) == [0, 1, 2, 3]
    assert [bm.allocate() for _ in range(4)] == [3, 2, 1, 0]
    assert bm.allocate() == -1
    bm.free(2)
    bm.free(0)
    assert list(bm.free_blocks) == [2, 0]
    assert bm.allocate() == 0


class ListEngine:
    """The engine's code on Python lists: one token at a time (decode, :1984-2001;
    verify, :3011-3023) with `while` growth, retire frees table[0..len) ascending
    (:3626-3628), rollback keeps ceil(len/bs) blocks and frees the tail ascending."""

    def __init__(self, num_blocks, bs, nseq, kv_stride):
        self.free = list(range(num_blocks))
        self.bs = bs
        self.tables = [[] for _ in range(nseq)]
        self.rows = {}  # (row) -> (k tuple)
        self.kv_stride = kv_stride

    def alloc(self):
        return self.free.pop() if self.free else -1

    def append(self, s, pos, kvecs):
        for b in range(len(kvecs)):
            p = pos + b
            while p // self.bs >= len(self.tables[s]):
                blk = self.alloc()
                if blk < 0:
                    return -1
                self.tables[s].append(blk)
        for b, k in enumerate(kvecs):
            p = pos + b
            self.rows[self.tables[s][p // self.bs] * self.bs + p % self.bs] = k
        return 0

    def rollback(self, s, new_len):
        keep = min(len(self.tables[s]), -(-new_len // self.bs))
        for blk in self.tables[s][keep:]:
            self.free.append(blk)
        del self.tables[s][keep:]


def _check_partition(st, nseq, num_blocks):
    used = [int(b) for s in range(nseq) for b in st.tables[s, :st.table_lens[s]]]
    free = [int(b) for b in st.free_list]
    assert sorted(used + free) == list(range(num_blocks)), "blocks not partitioned"


@pytest.mark.parametrize("seed", range(6))
def test_append_rollback_matches_list_engine(seed):
    rng = np.random.default_rng(seed)
    nseq, bs, num_blocks, kvs, stride = 5, 4, 24, 8, 16
    st = O.CacheState(1, kvs, bs, num_blocks, nseq, stride)
    eng = ListEngine(num_blocks, bs, nseq, kvs)
    length = [0] * nseq
    for step in range(60):
        op = rng.integers(0, 3)
        if op < 2:  # append a ragged batch
            n_new = rng.integers(0, 6, nseq).astype(np.int32)
            pos = np.array(length, np.int32)
            off = O.ragged_tok_off(n_new)
            k = rng.standard_normal((int(off[-1]) + 1, kvs)).astype(np.float32)
            v = rng.standard_normal((int(off[-1]) + 1, kvs)).astype(np.float32)
            status = st.append(0, pos, off, k, v, 5)
            for s in range(nseq):
                if n_new[s] == 0:
                    assert status[s] == 0
                    continue
                rc = eng.append(s, length[s], [tuple(k[off[s] + b]) for b in range(n_new[s])])
                assert status[s] == rc, (step, s)
                if rc == 0:
                    length[s] += int(n_new[s])
        else:  # accept a prefix / retire
            new_len = np.full(nseq, -1, np.int32)
            for s in range(nseq):
                if rng.random() < 0.5:
                    nl = int(rng.integers(0, length[s] + 1))
                    new_len[s] = nl
                    eng.rollback(s, nl)
                    length[s] = nl
            st.rollback(new_len)
        for s in range(nseq):
            assert list(st.tables[s, :st.table_lens[s]]) == eng.tables[s], (step, s)
        assert list(st.free_list) == eng.free, step
        _check_partition(st, nseq, num_blocks)
    # Rows of every live token hold the exact appended vector.
    for s in range(nseq):
        for p in range(length[s]):
            row = eng.tables[s][p // bs] * bs + p % bs
            np.testing.assert_array_equal(st.k_pools[0][row * kvs:(row + 1) * kvs],
                                          np.array(eng.rows[row], np.float32))


def test_decode_append_allocates_on_block_boundary_only():
    st = O.CacheState(1, 4, 16, 8, 1, 8)
    k = np.ones((1, 1, 4), np.float32)
    for p in range(33):
        st.append(0, [p], [0, 1], k * p, k * -p, 1)
        assert st.table_lens[0] == p // 16 + 1
    # LIFO: first allocation is the last block (max-1), then max-2, ...
    assert list(st.tables[0, :3]) == [7, 6, 5]
    assert list(st.free_list) == [0, 1, 2, 3, 4]
    row = 5 * 16 + 0  # token 32 lives in block 5, slot 0
    np.testing.assert_array_equal(st.k_pools[0][row * 4:(row + 1) * 4], np.full(4, 32.0))
    np.testing.assert_array_equal(st.v_pools[0][row * 4:(row + 1) * 4], np.full(4, -32.0))


def test_out_of_blocks_keeps_popped_blocks_and_writes_nothing():
    # verify-style multi-token append that runs out mid-way (…batched.mojo:3011-3023)
    st = O.CacheState(1, 4, 4, 3, 2, 8)
    k = np.arange(16 * 4, dtype=np.float32).reshape(16, 4)
    status = st.append(0, [0, 0], [0, 4, 16], k, k, 12)
    assert list(status) == [0, -1]
    assert list(st.tables[0, :1]) == [2]
    assert list(st.tables[1, :st.table_lens[1]]) == [1, 0]  # popped before the list ran dry
    assert st.bm.count[0] == 0
    # none of sequence 1's rows was written
    for blk in (1, 0):
        assert np.all(st.k_pools[0][blk * 16:(blk + 1) * 16] == 0)
    # decode append for seq 0 into its partially filled block still works
    status = st.append(0, [4, -1], [0, 0, 0], k, k, 12)
    assert list(status) == [0, 0]
    # a token range beyond the new rows, or longer than max_new, is rejected unchanged
    status = st.append(0, [3, 0], [0, 1, 17], k, k, 12)
    assert list(status) == [0, -5]
    status = st.append(0, [5, 0], [0, 13, 14], k, k, 12)
    assert list(status) == [-5, 0]  # seq 1 writes into a block it already holds


def test_table_full_is_reported_and_changes_nothing():
    st = O.CacheState(1, 4, 4, 16, 1, 2)
    k = np.ones((9, 4), np.float32)
    status = st.append(0, [0], [0, 9], k, k, 9)  # needs 3 blocks, table holds 2
    assert list(status) == [-2]
    assert st.table_lens[0] == 0 and st.bm.count[0] == 16


def test_rollback_semantics():
    st = O.CacheState(1, 4, 16, 16, 2, 8)
    k = np.zeros((73, 4), np.float32)
    st.append(0, [0, 0], [0, 40, 73], k, k, 40)
    assert list(st.table_lens) == [3, 3]
    t0, t1 = list(st.tables[0, :3]), list(st.tables[1, :3])
    st.rollback([32, 17])  # keep ceil(32/16)=2 and ceil(17/16)=2
    assert list(st.table_lens) == [2, 2]
    # freed in ascending logical order, sequence order: seq0's block 2 then seq1's block 2
    assert list(st.free_list[-2:]) == [t0[2], t1[2]]
    st.rollback([-1, 0])  # retire seq 1: frees its table ascending
    assert list(st.free_list[-2:]) == t1[:2]
    assert st.table_lens[1] == 0 and st.table_lens[0] == 2


def test_rollback_then_reappend_matches_fresh_run():
    # a16 invariant: rejected drafts rolled back, then re-appended, give the same table as
    # a run that never appended them (same free-list state).
    bs = 16
    a = O.CacheState(1, 4, bs, 64, 1, 16)
    b = O.CacheState(1, 4, bs, 64, 1, 16)
    k = np.zeros((200, 4), np.float32)
    a.append(0, [0], [0, 30], k, k, 200)
    b.append(0, [0], [0, 30], k, k, 200)
    a.append(0, [30], [0, 4], k, k, 200)  # draft crosses into a third block
    a.rollback([31])  # accept 1 -> back to 2 blocks
    b.append(0, [30], [0, 1], k, k, 200)
    np.testing.assert_array_equal(a.table_lens, b.table_lens)
    np.testing.assert_array_equal(a.tables[0, :a.table_lens[0]], b.tables[0, :b.table_lens[0]])
    np.testing.assert_array_equal(a.free_list[:-1], b.free_list[:-1])
    # a holds the freed block on top of its free list; the next allocation takes it back
    a.append(0, [31], [0, 10], k, k, 200)
    b.append(0, [31], [0, 10], k, k, 200)
    assert a.table_lens[0] == b.table_lens[0] == 3
