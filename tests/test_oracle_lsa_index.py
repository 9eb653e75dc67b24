"""CPU checks that pin the oracle's restatement of LSALayerIndex.reset / rollback_to
(lsa_core.mojo:281-303): the reference's rollback test (test_spec_verify_and_coalesce.mojo:
17-66) restated on the index's integer state, and closed forms of the state machine.

append_key (lsa_core.mojo:305-323) is modelled here only for its effect on that state: a
token at pos < max_capacity is counted, and the token at pos % 512 == 511 closes the block
(ward_cluster_block, :325-518), which fills the block's 32 bucket counts and increments
closed_blocks unless the block lies past max_buckets. The counts a closed block receives come
from Ward clustering in the reference; here they are a deterministic function of the keys,
which is all the rollback and replay checks need."""
import numpy as np

from oracle import oracle as O


def _append(st: O.LsaIndexState, pos: int, key_seed: int):
    if pos >= st.max_capacity:
        return
    st.total_tokens[0] += 1
    if pos % 512 == 511:
        b = int(st.closed_blocks[0])
        if (b + 1) * 32 > st.max_buckets:
            return
        rng = np.random.default_rng(key_seed * 1000003 + b)
        labels = rng.integers(0, 32, 128)  # one label per pool of 4 tokens
        counts = np.minimum(np.bincount(labels, minlength=32) * 4, 32)
        st.sizes[b * 32:(b + 1) * 32] = counts
        st.closed_blocks[0] += 1


def _state(st):
    return int(st.closed_blocks[0]), int(st.total_tokens[0]), st.sizes.copy()


def test_reference_rollback_across_and_at_the_block_boundary():
    # test_spec_verify_and_coalesce.mojo:17-66, max_capacity 2048.
    clean, spec = O.LsaIndexState(2048), O.LsaIndexState(2048)
    for pos in range(515):
        _append(clean, pos, 1)
        if pos < 510:
            _append(spec, pos, 1)
    for pos in range(510, 515):  # bogus drafts 510..514 close block 0 with other keys
        _append(spec, pos, 2)
    assert spec.closed_blocks[0] == 1
    spec.rollback_to(510)
    assert spec.closed_blocks[0] == 0 and spec.total_tokens[0] == 510
    assert np.all(spec.sizes[:32] == 0)
    for pos in range(510, 515):
        _append(spec, pos, 1)
    c1, t1, s1 = _state(spec)
    c2, t2, s2 = _state(clean)
    assert (c1, t1) == (c2, t2) == (1, 515)
    np.testing.assert_array_equal(s1, s2)
    spec.rollback_to(512)  # exact boundary: block 0 stays closed
    assert spec.closed_blocks[0] == 1 and spec.total_tokens[0] == 512
    np.testing.assert_array_equal(spec.sizes, s2)


def test_reset_for_non_positive_targets():
    for target in (0, -1, -1000):
        st = O.LsaIndexState(4096)
        for pos in range(1500):
            _append(st, pos, 3)
        assert st.closed_blocks[0] == 2
        st.rollback_to(target)
        assert st.closed_blocks[0] == 0 and st.total_tokens[0] == 0
        assert not st.sizes.any()


def test_rollback_within_a_block_keeps_every_bucket():
    st = O.LsaIndexState(4096)
    for pos in range(700):
        _append(st, pos, 4)
    before = st.sizes.copy()
    st.rollback_to(600)
    assert st.closed_blocks[0] == 1 and st.total_tokens[0] == 600
    np.testing.assert_array_equal(st.sizes, before)
    st.rollback_to(650)  # a later target only sets the count (the reference does the same)
    assert st.closed_blocks[0] == 1 and st.total_tokens[0] == 650


def test_two_blocks_reopen_and_capacity_clamps():
    st = O.LsaIndexState(2048)
    for pos in range(1600):
        _append(st, pos, 5)
    assert st.closed_blocks[0] == 3
    st.rollback_to(1000)  # 1000 // 512 = 1: blocks 1 and 2 reopen
    assert st.closed_blocks[0] == 1 and st.total_tokens[0] == 1000
    assert st.sizes[:32].any() and not st.sizes[32:].any()
    st2 = O.LsaIndexState(2048)
    for pos in range(2100):  # positions >= max_capacity are not counted
        _append(st2, pos, 6)
    assert st2.total_tokens[0] == 2048 and st2.closed_blocks[0] == 4
    before = st2.sizes.copy()
    st2.rollback_to(5000)
    assert st2.total_tokens[0] == 2048 and st2.closed_blocks[0] == 4
    np.testing.assert_array_equal(st2.sizes, before)


def test_rollback_then_replay_equals_a_clean_run_at_every_boundary():
    # For every rollback target around the block edges, replaying the true keys from the
    # target reproduces the state of a run that never saw the drafts.
    for target in (1, 510, 511, 512, 513, 1023, 1024, 1025, 1030):
        clean, spec = O.LsaIndexState(4096), O.LsaIndexState(4096)
        for pos in range(1030):
            _append(clean, pos, 7)
            if pos < target:
                _append(spec, pos, 7)
        for pos in range(target, target + 8):
            _append(spec, pos, 8)  # drafts with other keys
        spec.rollback_to(target)
        for pos in range(target, 1030):
            _append(spec, pos, 7)
        a, b = _state(spec), _state(clean)
        assert a[:2] == b[:2], target
        np.testing.assert_array_equal(a[2], b[2])
