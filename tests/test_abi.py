"""CPU checks of the C ABI: libpkv.so loads and exports every symbol include/pkv.h
declares; argument validation runs host-side (no device call is made)."""
import ctypes
import os
import re

import pytest

from pkv import lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "pkv.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = lib.load()
    names = declared_symbols()
    assert "pkv_append" in names and "pkv_attend" in names and "pkv_rollback" in names
    for n in names:
        assert hasattr(L, n), f"{n} declared in pkv.h but not exported"
    assert set(names) == set(lib.PROTOTYPES), "ctypes prototypes out of sync with pkv.h"


def test_version_and_error_string():
    L = lib.load()
    assert L.pkv_version() >> 16 == 1
    assert isinstance(L.pkv_last_error(), bytes)


def _params(**kw):
    p = lib.PkvParams()
    vals = dict(num_heads=16, num_kv_heads=8, head_dim=256, block_size=16, num_blocks=64,
                window=0, scale=1.0, kv_dtype=0, ring_size=0, reserved=0)
    vals.update(kw)
    for k, v in vals.items():
        setattr(p, k, v)
    return p


def test_workspace_size_is_monotone_and_validates():
    L = lib.load()
    p = _params()
    a = L.pkv_workspace_size(ctypes.byref(p), 32, 1, 8192)
    b = L.pkv_workspace_size(ctypes.byref(p), 32, 1, 32768)
    assert 0 < a < b
    w = _params(window=1024)
    assert L.pkv_workspace_size(ctypes.byref(w), 32, 1, 32768) < b  # window bounds the chunks
    ring = _params(window=1024, ring_size=1032)
    assert 0 < L.pkv_workspace_size(ctypes.byref(ring), 32, 1, 32768) \
        <= L.pkv_workspace_size(ctypes.byref(w), 32, 1, 32768)
    for bad in (_params(num_kv_heads=3), _params(head_dim=100), _params(ring_size=-8),
                _params(kv_dtype=7), _params(block_size=0)):
        assert L.pkv_workspace_size(ctypes.byref(bad), 1, 1, 10) == 0


@pytest.mark.parametrize("kw,code", [
    (dict(num_kv_heads=3), lib.PKV_ERR_INVALID),
    (dict(head_dim=96), lib.PKV_ERR_UNSUPPORTED),
    (dict(ring_size=-1), lib.PKV_ERR_INVALID),
])
def test_invalid_params_rejected_before_launch(kw, code):
    L = lib.load()
    p = _params(**kw)
    rc = L.pkv_attend(None, ctypes.byref(p), 1, 1, 1, 1, 4, 1, 1, 1, 10, 1, 1, 1 << 20)
    assert rc == code
    assert L.pkv_last_error()


def test_null_pointers_and_small_workspace_rejected():
    L = lib.load()
    p = _params()
    assert L.pkv_attend(None, ctypes.byref(p), None, 1, 1, 1, 4, 1, 1, 1, 10, 1, 1, 1 << 20) \
        == lib.PKV_ERR_INVALID
    assert L.pkv_attend(None, ctypes.byref(p), 1, 1, 1, 1, 4, 1, 1, 1, 10, 1, 1, 16) \
        == lib.PKV_ERR_WORKSPACE
    assert L.pkv_rollback(None, ctypes.byref(p), None, 4, 1, 1, 1, 1, 1, None) \
        == lib.PKV_ERR_INVALID
    assert L.pkv_append(None, ctypes.byref(p), 1, 1, 1, 4, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, None) \
        == lib.PKV_ERR_INVALID
    assert L.pkv_append(None, ctypes.byref(p), 1, 1, 1, 4, 1, 1, 1, 1, 1, 1, 1, 1, 1, 5000, 1) \
        == lib.PKV_ERR_UNSUPPORTED
    # head_dim 64 (no stream kernel) with too many query rows per kv head (9 x 2 > 16)
    d64 = _params(head_dim=64)
    assert L.pkv_attend(None, ctypes.byref(d64), 1, 1, 1, 1, 4, 1, 9, 1, 10, 1, 1, 1 << 30) \
        == lib.PKV_ERR_UNSUPPORTED


def test_ring_mode_rejections():
    """Ring pools: prefill and rollback refuse them, the single-sequence drop-in checks
    ring_base against the pool and the window against the ring (the reference aborts,
    attention.mojo:265-266) -- all before any launch."""
    L = lib.load()
    ring = _params(window=1024, ring_size=1032, kv_dtype=1, num_blocks=4)
    assert L.pkv_prefill(None, ctypes.byref(ring), 1, 1, 1, 1, 4, 1, 1, 16, 1, 100, 1) \
        == lib.PKV_ERR_UNSUPPORTED
    assert L.pkv_rollback(None, ctypes.byref(ring), 1, 4, 1, 1, 1, 1, 1, None) \
        == lib.PKV_ERR_INVALID
    # (stream, q, k, v, table, bs, pos, hq, hkv, d, window, out, ring_size, ring_base,
    #  num_blocks, dtype, ws, ws_bytes)
    args = [None, 1, 1, 1, None, 16, 2000, 16, 8, 256, 1024, 1, 1032, 0, 4, 0, 1, 1 << 30]
    bad_base = list(args)
    bad_base[13] = 3 * 1032 + 1  # ring would end past the 4 rings of the pool
    assert L.pkv_paged_attention_layer(*bad_base) == lib.PKV_ERR_INVALID
    small_ring = list(args)
    small_ring[12] = 1000  # window 1024 > ring 1000
    assert L.pkv_paged_attention_layer(*small_ring) == lib.PKV_ERR_INVALID
    full_causal = list(args)
    full_causal[10] = 0  # pos 2000 with no window: 2001 keys > ring
    assert L.pkv_paged_attention_layer(*full_causal) == lib.PKV_ERR_INVALID


def test_prefill_block_size_below_8_rejected_before_launch():
    """The prefill kernel copies each wave's eight keys of a tile from one block."""
    L = lib.load()
    small = _params(kv_dtype=1, block_size=4, num_blocks=64)
    assert L.pkv_prefill(None, ctypes.byref(small), 1, 1, 1, 1, 4, 1, 1, 16, 1, 100, 1) \
        == lib.PKV_ERR_UNSUPPORTED
    assert b"block_size" in L.pkv_last_error()


def test_q4_matmul_rejections_before_launch():
    L = lib.load()
    assert L.pkv_q4_matmul(None, 16, 4, 16, 100, 8, 1, 16, 16, 1 << 20) == lib.PKV_ERR_INVALID
    assert L.pkv_q4_matmul(None, 16, 4, 16, 128, 8, 65, 16, 16, 1 << 20) == lib.PKV_ERR_UNSUPPORTED
    assert L.pkv_q4_matmul(None, 16, 4, 16, 4096, 8, 8, 16, 16, 16) == lib.PKV_ERR_WORKSPACE
    assert L.pkv_q4_matmul(None, 16, 4, 8, 4096, 8, 8, 16, 16, 1 << 20) == lib.PKV_ERR_INVALID  # x alignment
    assert L.pkv_q4_matmul(None, 4, 4, 16, 4096, 8, 8, 16, 16, 1 << 20) == lib.PKV_ERR_INVALID  # w alignment
    # 22 row groups' arrival counts (one 256-byte line), then partials of up to 512
    # workgroups of 128 rows
    assert L.pkv_q4_matmul_workspace_size(4096, 2816, 32) == 256 + 512 * 32 * 128 * 4


def test_lsa_cache_rejections_before_launch():
    L = lib.load()
    assert L.pkv_lsa_max_keys(64, 4, 16) == 84
    assert L.pkv_lsa_max_keys(0, 4, 16) == 21 and L.pkv_lsa_max_keys(-3, -1, -1) == 1
    assert L.pkv_lsa_max_keys(2**31 - 1, 2**31 - 1, 1) == -1
    p = 16  # a stand-in non-null address; none of these calls reaches a launch
    args = dict(ids=p, picked=p, stride=8, npk=p, pos=p, top_k=64, sink=4, window=16, batch=4,
                sizes=p, members=p, nidx=6, maxb=128, keys=p, off=p, cap=4 * 84, status=p,
                ws=p, ws_bytes=(4 * 84 + 4) * 4)
    assert L.pkv_lsa_expand_workspace_size(4, 64, 4, 16) == (4 * 84 + 4) * 4
    assert L.pkv_lsa_expand_workspace_size(0, 64, 4, 16) == 0

    def expand(**kw):
        a = {**args, **kw}
        return L.pkv_lsa_expand(None, a["ids"], a["picked"], a["stride"], a["npk"], a["pos"],
                                a["top_k"], a["sink"], a["window"], a["batch"], a["sizes"],
                                a["members"], a["nidx"], a["maxb"], a["keys"], a["off"],
                                a["cap"], a["status"], a["ws"], a["ws_bytes"])
    assert expand(batch=0) == lib.PKV_ERR_INVALID
    assert expand(batch=1025) == lib.PKV_ERR_UNSUPPORTED
    assert expand(keys=None) == lib.PKV_ERR_INVALID
    assert expand(window=-1) == lib.PKV_ERR_INVALID
    assert expand(nidx=0) == lib.PKV_ERR_INVALID
    assert expand(cap=4 * 84 - 1) == lib.PKV_ERR_WORKSPACE
    assert expand(ws_bytes=(4 * 84 + 4) * 4 - 1) == lib.PKV_ERR_WORKSPACE
    assert expand(ws=None) == lib.PKV_ERR_INVALID
    assert L.pkv_lsa_rollback(None, p, p, 3, 6, 2048, 100, p, p, p) == lib.PKV_ERR_INVALID
    assert L.pkv_lsa_rollback(None, p, p, -1, 6, 2048, 128, p, p, p) == lib.PKV_ERR_INVALID
    assert L.pkv_lsa_rollback(None, None, p, 3, 6, 2048, 128, p, p, p) == lib.PKV_ERR_INVALID
    assert L.pkv_lsa_rollback(None, None, None, 0, 6, 2048, 128, None, None, None) == lib.PKV_OK


def test_verify_rejections_before_launch():
    L = lib.load()
    p = _params()
    import ctypes
    ptr = 16
    # q_lens is required; a geometry without the stream path cannot take per-sequence counts
    assert L.pkv_verify(None, ctypes.byref(p), ptr, ptr, ptr, ptr, 8, ptr, None, 4, 2, 100, ptr,
                        ptr, 1 << 20) == lib.PKV_ERR_INVALID
    p64 = _params(head_dim=64)
    assert L.pkv_verify(None, ctypes.byref(p64), ptr, ptr, ptr, ptr, 8, ptr, ptr, 4, 2, 100, ptr,
                        ptr, 1 << 20) == lib.PKV_ERR_UNSUPPORTED


def test_append_attend_rejections_before_launch():
    # The fused step checks the attention's arguments, then the append's, before any launch.
    L = lib.load()
    p = _params()
    ptr = 16
    ws = L.pkv_workspace_size(ctypes.byref(p), 4, 1, 100)

    def call(q=ptr, q_len=1, ws_bytes=ws, k_new=ptr, status=ptr, batch=4, max_pos=100):
        return L.pkv_append_attend(None, ctypes.byref(p), ptr, ptr, ptr, 8, ptr, ptr, ptr, ptr,
                                   ptr, 1, k_new, ptr, 4, status, q, q_len, batch, max_pos, ptr,
                                   ptr, ws_bytes)

    assert call(q=None) == lib.PKV_ERR_INVALID
    assert call(q_len=0) == lib.PKV_ERR_INVALID
    assert call(max_pos=-1) == lib.PKV_ERR_INVALID
    assert call(batch=5000) == lib.PKV_ERR_INVALID
    assert call(ws_bytes=ws - 1) == lib.PKV_ERR_WORKSPACE
    assert call(k_new=None) == lib.PKV_ERR_INVALID
    assert call(status=None) == lib.PKV_ERR_INVALID
