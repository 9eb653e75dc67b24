"""Writes the golden fixtures of the paged KV path at tiny scale (run from the repository
root: python tests/golden/make_fixtures.py).

Each fixture is an .npz (no pickled objects) holding the seed, the geometry and a SHA-256
of the inputs the generator below draws from that seed, and the expected results the
oracle (oracle/pkv_oracle.c) computes from them: block tables, table lengths, free lists
and counts, SHA-256 of the pools after every append, and the attention outputs (the
oracle's fp32 path and its float64 path, both stored as fp32).

  config1_tiny: the shape of BASELINE config 1 (a single sequence whose append takes a
    new block from the back of the LIFO free list, then attends over every key), with
    4 q / 2 kv heads, head_dim 256, a 4-block table and 16 blocks in the pool.
  config5_tiny: the shape of config 5 (MTP reads of the shared pool at pos - 1, a 4-token
    verify append + causal attention, acceptance of 0..4 drafts, rollback), 3 sequences,
    2 q / 1 kv head, head_dim 256, 3 iterations.

Inputs are drawn with numpy.random.default_rng(seed) in the order the functions below draw
them; tests regenerate them the same way and check the stored input hash first.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402

BS = 16
SCALE = 0.0625


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def config1_inputs(seed=101):
    g = dict(HQ=4, HKV=2, D=256, NB=16, STRIDE=8, PREFIX=4, POS=64)
    rng = np.random.default_rng(seed)
    kvs = g["HKV"] * g["D"]
    perm = rng.permutation(g["NB"]).astype(np.int32)
    k = rng.standard_normal(g["NB"] * BS * kvs, dtype=np.float32)
    v = rng.standard_normal(g["NB"] * BS * kvs, dtype=np.float32)
    q = rng.standard_normal((1, 1, g["HQ"], g["D"]), dtype=np.float32)
    k_new = rng.standard_normal((1, kvs), dtype=np.float32)
    v_new = rng.standard_normal((1, kvs), dtype=np.float32)
    table = perm[:g["PREFIX"]]
    free = np.sort(perm[g["PREFIX"]:])  # the unused ids in ascending order
    return g, dict(table=table, free=free, k=k, v=v, q=q, k_new=k_new, v_new=v_new)


def config1_state(g, x):
    st = O.CacheState(1, g["HKV"] * g["D"], BS, g["NB"], 1, g["STRIDE"])
    st.k_pools[0][:] = x["k"]
    st.v_pools[0][:] = x["v"]
    st.tables[0, :g["PREFIX"]] = x["table"]
    st.table_lens[0] = g["PREFIX"]
    st.bm.free_list[:x["free"].size] = x["free"]
    st.bm.count[0] = x["free"].size
    return st


def config1_expected(g, x):
    st = config1_state(g, x)
    pos = np.array([g["POS"]], np.int32)
    status = st.append(0, pos, [0, 1], x["k_new"], x["v_new"], 1)
    ref = O.attend(x["q"], st.k_pools[0], st.v_pools[0], st.tables, st.table_lens, pos, 1,
                   g["HQ"], g["HKV"], g["D"], BS, 0, scale=SCALE)
    exact = O.attend_f64(x["q"], st.k_pools[0], st.v_pools[0], st.tables, pos, 1, g["HQ"],
                         g["HKV"], g["D"], BS, 0, scale=SCALE)
    return dict(status=status, tables=st.tables.copy(), table_lens=st.table_lens.copy(),
                free_list=st.free_list, k_sha=sha(st.k_pools[0]), v_sha=sha(st.v_pools[0]),
                out_ref=ref.astype(np.float32), out_exact=exact.astype(np.float32))


def config5_inputs(seed=505):
    g = dict(HQ=2, HKV=1, D=256, NB=40, STRIDE=12, B=3, DRAFT=4, ITERS=3)
    rng = np.random.default_rng(seed)
    kvs = g["HKV"] * g["D"]
    ctx = np.array([40, 77, 100], np.int32)
    perm = rng.permutation(g["NB"]).astype(np.int32)
    k = rng.standard_normal(g["NB"] * BS * kvs, dtype=np.float32)
    v = rng.standard_normal(g["NB"] * BS * kvs, dtype=np.float32)
    its = []
    for _ in range(g["ITERS"]):
        its.append(dict(
            q_mtp=rng.standard_normal((g["B"], 1, g["HQ"], g["D"]), dtype=np.float32),
            q=rng.standard_normal((g["B"], g["DRAFT"], g["HQ"], g["D"]), dtype=np.float32),
            k_new=rng.standard_normal((g["B"] * g["DRAFT"], kvs), dtype=np.float32),
            v_new=rng.standard_normal((g["B"] * g["DRAFT"], kvs), dtype=np.float32),
            accept=rng.integers(0, g["DRAFT"] + 1, g["B"]).astype(np.int32)))
    # tables hold exactly the blocks of positions < ctx; the rest of the pool is free
    need = (ctx + BS - 1) // BS
    tables = np.zeros((g["B"], g["STRIDE"]), np.int32)
    o = 0
    for s in range(g["B"]):
        tables[s, :need[s]] = perm[o:o + need[s]]
        o += need[s]
    free = np.sort(perm[o:])
    return g, dict(ctx=ctx, tables=tables, lens=need.astype(np.int32), free=free, k=k, v=v,
                   its=its)


def config5_input_arrays(x):
    out = [x["ctx"], x["tables"], x["lens"], x["free"], x["k"], x["v"]]
    for it in x["its"]:
        out += [it["q_mtp"], it["q"], it["k_new"], it["v_new"], it["accept"]]
    return out


def config5_state(g, x):
    st = O.CacheState(1, g["HKV"] * g["D"], BS, g["NB"], g["B"], g["STRIDE"])
    st.k_pools[0][:] = x["k"]
    st.v_pools[0][:] = x["v"]
    st.tables[:] = x["tables"]
    st.table_lens[:] = x["lens"]
    st.bm.free_list[:x["free"].size] = x["free"]
    st.bm.count[0] = x["free"].size
    return st


def config5_expected(g, x):
    """Per iteration: the MTP read at pos - 1 (read only), the verify append of DRAFT rows
    per sequence and DRAFT causal queries, then rollback to pos + accept (the accepted
    drafts stay, the rest of the appended blocks go back to the free list)."""
    st = config5_state(g, x)
    pos = x["ctx"].copy()
    DR = g["DRAFT"]
    res = dict(tables=[], table_lens=[], free_list=[], k_sha=[], v_sha=[], status=[])
    for i, it in enumerate(x["its"]):
        last = i == len(x["its"]) - 1
        if last:
            res["mtp_ref"] = O.attend(it["q_mtp"], st.k_pools[0], st.v_pools[0], st.tables,
                                      st.table_lens, pos - 1, 1, g["HQ"], g["HKV"], g["D"], BS,
                                      0, scale=SCALE).astype(np.float32)
            res["mtp_exact"] = O.attend_f64(it["q_mtp"], st.k_pools[0], st.v_pools[0],
                                            st.tables, pos - 1, 1, g["HQ"], g["HKV"], g["D"],
                                            BS, 0, scale=SCALE).astype(np.float32)
        tok_off = O.dense_tok_off(g["B"], DR)
        res["status"].append(st.append(0, pos, tok_off, it["k_new"], it["v_new"], DR))
        if last:
            res["verify_ref"] = O.attend(it["q"], st.k_pools[0], st.v_pools[0], st.tables,
                                         st.table_lens, pos, DR, g["HQ"], g["HKV"], g["D"], BS,
                                         0, scale=SCALE).astype(np.float32)
            res["verify_exact"] = O.attend_f64(it["q"], st.k_pools[0], st.v_pools[0], st.tables,
                                               pos, DR, g["HQ"], g["HKV"], g["D"], BS, 0,
                                               scale=SCALE).astype(np.float32)
        pos = pos + it["accept"]
        st.rollback(pos)
        res["tables"].append(st.tables.copy())
        res["table_lens"].append(st.table_lens.copy())
        fl = np.full(g["NB"], -1, np.int32)
        fl[:st.free_list.size] = st.free_list
        res["free_list"].append(fl)
        res["k_sha"].append(sha(st.k_pools[0]))
        res["v_sha"].append(sha(st.v_pools[0]))
    out = {k: (np.array(v) if k.endswith("_sha") else np.stack(v)) if isinstance(v, list) else v
           for k, v in res.items()}
    out["final_pos"] = pos
    return out


def main():
    g1, x1 = config1_inputs()
    e1 = config1_expected(g1, x1)
    np.savez(os.path.join(HERE, "config1_tiny.npz"), seed=101,
             input_sha=sha(x1["table"], x1["free"], x1["k"], x1["v"], x1["q"], x1["k_new"],
                           x1["v_new"]),
             **{f"geom_{k}": v for k, v in g1.items()},
             **{k: (np.array(v) if isinstance(v, str) else v) for k, v in e1.items()})
    g5, x5 = config5_inputs()
    e5 = config5_expected(g5, x5)
    np.savez(os.path.join(HERE, "config5_tiny.npz"), seed=505,
             input_sha=sha(*config5_input_arrays(x5)),
             **{f"geom_{k}": v for k, v in g5.items()}, **e5)
    for n in ("config1_tiny.npz", "config5_tiny.npz"):
        print(n, os.path.getsize(os.path.join(HERE, n)), "bytes")


if __name__ == "__main__":
    main()
