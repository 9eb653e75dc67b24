"""GPU parity of BASELINE.json config 2 -- the headline benchmark workload -- through the
exact call bench.py times, against the oracle's restatement of the reference CPU path.

The full 64-step schedule of pkv.workloads.DecodeSchedule(seed=0): 32 sequences with
contexts U[128, 8192] on a sliding-window (1024) layer and a global layer, 16q / 8kv /
256, block 16, fp32 pools; every step appends one token per sequence and attends on both
layers through one pkv_append_attend call per layer (the append into partially filled
blocks, the block allocation from the LIFO free list, and the attention, whose launch
also writes the appended rows); every 8th step first retires 4 sequences (pkv_rollback
to length 0, blocks freed in ascending order, model_speculative_moe_batched.mojo
:3602-3637) and admits 4 new 256-token contexts into the freed blocks (pkv_append).
The oracle replays the same calls on its own state (appends :1984-2001, attention
attention.mojo:240-294).

Checked:
  - after every call: per-sequence status, block tables, table lengths and the free list,
    bit-exact;
  - at every retire/admit event and after the last step: all four pools, bit-exact;
  - every step's outputs on both layers against the oracle's fp32 path and against the
    float64 attention, by the parity rule of tests/parity.py. The test prints the largest
    error against the fp32 reference next to the literal 1e-4 bound, together with that
    reference's own distance from the float64 attention (on these long contexts the fp32
    reference itself sits ~1.2e-4 from exact; the GPU accumulates in double).

test_engine_global512_schedule_append_attend runs the same schedule on the engine's
global-layer geometry (16q / 2kv / 512, one full-attention layer): bench.py --leg
global512."""
import numpy as np
import pytest

from oracle import oracle as O
from pkv import LayerSpec, PagedKVCache, hip
from pkv.workloads import DecodeSchedule
from tests import parity

pytestmark = pytest.mark.gpu


def _compare_state(cache, st, what):
    snap = cache.snapshot()
    assert np.array_equal(snap["table_lens"], st.table_lens), f"{what}: table lengths differ"
    for s in range(st.tables.shape[0]):
        n = int(st.table_lens[s])
        assert np.array_equal(snap["tables"][s, :n], st.tables[s, :n]), \
            f"{what}: block table of sequence {s} differs"
    assert np.array_equal(snap["free_list"], st.free_list), f"{what}: free lists differ"


def _compare_pools(cache, st, what):
    for layer in range(len(cache.k_pools)):
        for name, dev, ref in (("K", cache.k_pools[layer], st.k_pools[layer]),
                               ("V", cache.v_pools[layer], st.v_pools[layer])):
            assert np.array_equal(dev.numpy().reshape(-1), ref), \
                f"{what}: layer {layer} {name} pool differs"


def _run_schedule(w, tag):
    """Every call of the schedule through the C ABI, replayed on the oracle's state."""
    B, L = w.B, w.L
    d = w.device_data()
    layers = [LayerSpec(w.HQ, w.HKV, w.D, window=win) for win in w.windows]
    cache = PagedKVCache(layers, block_size=w.BS, num_blocks=w.num_blocks, max_seqs=B,
                         max_blocks_per_seq=w.table_stride, max_q_len=1, max_pos=w.max_pos,
                         scale=w.SCALE)
    cache.tables.upload(w.tables0)
    cache.table_lens.upload(w.lens0)
    fl = np.zeros(w.num_blocks, np.int32)
    fl[:w.free0.size] = w.free0
    cache.free_list.upload(fl)
    cache.free_count.upload(np.array([w.free0.size], np.int32))
    st = O.CacheState(L, w.kv_stride, w.BS, w.num_blocks, B, w.table_stride, alloc_pools=False)
    st.tables[:] = w.tables0
    st.table_lens[:] = w.lens0
    st.bm.free_list[:w.free0.size] = w.free0
    st.bm.count[0] = w.free0.size
    for layer in range(L):
        cache.k_pools[layer].copy_from(d["pools"][layer][0])
        cache.v_pools[layer].copy_from(d["pools"][layer][1])
        st.k_pools[layer] = d["pools"][layer][0].numpy().reshape(-1)
        st.v_pools[layer] = d["pools"][layer][1].numpy().reshape(-1)
    qh, kh, vh = d["q"].numpy(), d["k_new"].numpy(), d["v_new"].numpy()
    ak, av = d["admit_k"].numpy(), d["admit_v"].numpy()
    row_bytes = w.kv_stride * 4
    qstep = B * w.HQ * w.D * 4
    kvstep = B * row_bytes
    dec_off = w.decode_tok_off()
    out = hip.DeviceArray((B, 1, w.HQ, w.D), np.float32)
    nthreads = O.max_threads()
    worst32, worst64, worst_own = 0.0, 0.0, 0.0
    for j in range(w.STEPS):
        if j in w.events:
            what = f"step {j} (retire {list(w.events[j])})"
            e = d["event_index"][j]
            nl = w.retire_new_len(j)
            rc = cache.rollback(nl).numpy()
            st.rollback(nl)
            assert np.all(rc == 0), f"{what}: rollback status {rc}"
            _compare_state(cache, st, f"{what} after rollback")
            for layer in range(L):
                base = (e * L + layer) * w.admit_rows * row_bytes
                sts = cache.append(layer, w.admit_pos(j), w.admit_tok_off(j),
                                   d["admit_k"].ptr + base, d["admit_v"].ptr + base,
                                   w.ADMIT_CTX, w.admit_rows).numpy()
                ref = st.append(layer, w.admit_pos(j), w.admit_tok_off(j), ak[e, layer],
                                av[e, layer], w.ADMIT_CTX)
                assert np.array_equal(sts, ref) and np.all(sts == 0), f"{what}: admit status"
                _compare_state(cache, st, f"{what} after admission, layer {layer}")
            _compare_pools(cache, st, what)
        for layer in range(L):
            window = w.windows[layer]
            what = f"step {j} layer {layer} ({'sliding' if window > 0 else 'global'})"
            off = j * L + layer
            sts = cache.append_attend(layer, w.pos[j], dec_off, d["k_new"].ptr + off * kvstep,
                                      d["v_new"].ptr + off * kvstep, 1, B,
                                      d["q"].ptr + off * qstep, 1, out).numpy()
            ref_st = st.append(layer, w.pos[j], dec_off, kh[j, layer], vh[j, layer], 1)
            assert np.array_equal(sts, ref_st) and np.all(sts == 0), f"{what}: status {sts}"
            _compare_state(cache, st, what)
            got = out.numpy()
            ref = O.attend(qh[j, layer], st.k_pools[layer], st.v_pools[layer], st.tables,
                           st.table_lens, w.pos[j], 1, w.HQ, w.HKV, w.D, w.BS, window,
                           scale=w.SCALE, nthreads=nthreads, par=1)
            exact = O.attend_f64(qh[j, layer], st.k_pools[layer], st.v_pools[layer],
                                 st.tables, w.pos[j], 1, w.HQ, w.HKV, w.D, w.BS, window,
                                 scale=w.SCALE)
            e32, e64 = parity.check(got, ref, exact, what=what)
            worst32, worst64 = max(worst32, e32), max(worst64, e64)
            worst_own = max(worst_own, O.max_rel_err(ref, exact))
        if j % 8 == 7:
            print(f"[{tag}] steps 0..{j} green: max rel err {worst32:.3g} vs the fp32 "
                  f"reference (literal bound {parity.TOL_F32:g}; that reference's own error "
                  f"vs float64 {worst_own:.3g}), {worst64:.3g} vs float64 (bound "
                  f"{parity.TOL_EXACT:g})", flush=True)
    _compare_pools(cache, st, "after the last step")
    print(f"[{tag}] {w.STEPS} steps x {L} layers: state and pools bit-exact; max rel err "
          f"{worst32:.3g} vs the fp32 reference (literal 1e-4; reference's own error "
          f"{worst_own:.3g}), {worst64:.3g} vs float64", flush=True)
    cache.free()


def test_config2_full_schedule_append_attend(gpu):
    print("[config2] building the 64-step schedule (seed 0)", flush=True)
    _run_schedule(DecodeSchedule(seed=0), "config2")


def test_engine_global512_schedule_append_attend(gpu):
    """The same 64-step schedule on the engine's global-layer geometry (16 q / 2 kv heads,
    head_dim 512, model_speculative_moe_batched.mojo:1905-1907; the MTP assistant's last
    layer reads that pool, :756-760): one full-attention fp32 layer, B = 32, contexts
    U[128, 8192], the bench's --leg global512 workload."""
    print("[global512] building the 64-step schedule (seed 0)", flush=True)
    _run_schedule(DecodeSchedule.engine_global(seed=0), "global512")
