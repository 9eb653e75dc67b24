"""The HIP path against the committed golden fixtures (tests/golden/*.npz) at tiny scale:
the same seeded inputs through libpkv's C ABI give the fixture's block tables, table
lengths, free lists and pool hashes bit for bit, and attention outputs within the parity
rule of tests/parity.py against the fixture's fp32 and float64 oracle outputs."""
import os

import numpy as np
import pytest

from pkv import F32, LayerSpec, PagedKVCache, hip
from tests import parity
from tests.golden import make_fixtures as F

pytestmark = pytest.mark.gpu

GOLDEN = os.path.dirname(F.__file__)


def _cache(g, B, q_len, x_tables, x_lens, free, k, v, max_pos):
    spec = LayerSpec(g["HQ"], g["HKV"], g["D"], window=0, kv_dtype=F32)
    cache = PagedKVCache([spec], block_size=F.BS, num_blocks=g["NB"], max_seqs=B,
                         max_blocks_per_seq=g["STRIDE"], max_q_len=q_len, max_pos=max_pos,
                         scale=F.SCALE)
    cache.tables.upload(x_tables)
    cache.table_lens.upload(x_lens)
    fl = np.zeros(g["NB"], np.int32)
    fl[:free.size] = free
    cache.free_list.upload(fl)
    cache.free_count.upload(np.array([free.size], np.int32))
    cache.k_pools[0].upload(k)
    cache.v_pools[0].upload(v)
    return cache


def _state_matches(cache, tables, lens, free, what):
    snap = cache.snapshot()
    assert np.array_equal(snap["table_lens"], lens), f"{what}: table lengths"
    for s in range(lens.size):
        n = int(lens[s])
        assert np.array_equal(snap["tables"][s, :n], tables[s, :n]), f"{what}: table {s}"
    assert np.array_equal(snap["free_list"], free), f"{what}: free list"


def test_config1_tiny_matches_fixture(gpu):
    print("[golden] config1_tiny", flush=True)
    fx = np.load(os.path.join(GOLDEN, "config1_tiny.npz"), allow_pickle=False)
    g, x = F.config1_inputs(int(fx["seed"]))
    tables = np.zeros((1, g["STRIDE"]), np.int32)
    tables[0, :g["PREFIX"]] = x["table"]
    cache = _cache(g, 1, 1, tables, np.array([g["PREFIX"]], np.int32), x["free"], x["k"],
                   x["v"], g["POS"])
    dk, dv = hip.DeviceArray.from_numpy(x["k_new"]), hip.DeviceArray.from_numpy(x["v_new"])
    pos = np.array([g["POS"]], np.int32)
    status = cache.append(0, pos, [0, 1], dk, dv, 1, 1).numpy()
    np.testing.assert_array_equal(status, fx["status"])
    _state_matches(cache, fx["tables"], fx["table_lens"], fx["free_list"], "config1")
    assert F.sha(cache.k_pools[0].numpy().reshape(-1)) == str(fx["k_sha"])
    assert F.sha(cache.v_pools[0].numpy().reshape(-1)) == str(fx["v_sha"])
    out = hip.DeviceArray((1, 1, g["HQ"], g["D"]), np.float32)
    cache.attend(0, hip.DeviceArray.from_numpy(x["q"]), pos, 1, out)
    parity.check(out.numpy(), fx["out_ref"], fx["out_exact"].astype(np.float64), what="config1")
    cache.free()


def test_config5_tiny_matches_fixture(gpu):
    print("[golden] config5_tiny", flush=True)
    fx = np.load(os.path.join(GOLDEN, "config5_tiny.npz"), allow_pickle=False)
    g, x = F.config5_inputs(int(fx["seed"]))
    B, DR = g["B"], g["DRAFT"]
    max_pos = g["STRIDE"] * F.BS - 1
    cache = _cache(g, B, DR, x["tables"], x["lens"], x["free"], x["k"], x["v"], max_pos)
    pos = x["ctx"].copy()
    tok_off = np.arange(B + 1, dtype=np.int32) * DR
    out_m = hip.DeviceArray((B, 1, g["HQ"], g["D"]), np.float32)
    out_v = hip.DeviceArray((B, DR, g["HQ"], g["D"]), np.float32)
    for i, it in enumerate(x["its"]):
        last = i == len(x["its"]) - 1
        cache.attend(0, hip.DeviceArray.from_numpy(it["q_mtp"]), pos - 1, 1, out_m)
        if last:
            parity.check(out_m.numpy(), fx["mtp_ref"], fx["mtp_exact"].astype(np.float64),
                         what="mtp")
        status = cache.append(0, pos, tok_off, hip.DeviceArray.from_numpy(it["k_new"]),
                              hip.DeviceArray.from_numpy(it["v_new"]), DR, B * DR).numpy()
        np.testing.assert_array_equal(status, fx["status"][i])
        cache.attend(0, hip.DeviceArray.from_numpy(it["q"]), pos, DR, out_v)
        if last:
            parity.check(out_v.numpy(), fx["verify_ref"], fx["verify_exact"].astype(np.float64),
                         what="verify")
        pos = pos + it["accept"]
        cache.rollback(pos)
        fl = fx["free_list"][i]
        _state_matches(cache, fx["tables"][i], fx["table_lens"][i], fl[fl >= 0], f"iteration {i}")
        assert F.sha(cache.k_pools[0].numpy().reshape(-1)) == str(fx["k_sha"][i])
        assert F.sha(cache.v_pools[0].numpy().reshape(-1)) == str(fx["v_sha"][i])
    np.testing.assert_array_equal(pos, fx["final_pos"])
    cache.free()
