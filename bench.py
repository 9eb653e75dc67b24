#!/usr/bin/env python3
"""Paged decode benchmark on one MI355X: BASELINE.json config 2 through libpkv's C ABI.

One step = one continuous-batching decode step of 32 sequences on a sliding-window
(1024) and a global layer (16 q / 8 kv heads, head_dim 256, block 16, fp32 pools):
per layer a fused K/V append (one token per sequence, into partially filled blocks)
and split-K paged attention; every 8th step first retires 4 sequences (their blocks go
back to the LIFO free list) and admits 4 new 256-token contexts into the freed blocks.
The 64-step schedule repeats; the small block-manager state is restored between
passes. Inputs (queries, new K/V rows, positions) are resident in HBM before timing.

Prints one JSON line. `roofline` covers the attention kernel (both layers' launches):
algorithmic bytes per launch (each attended K/V row slice once + Q + O + table
entries) over the average launch duration, timed with HIP events on the launch
stream. `cpu_baseline` times the reference CPU path (the oracle's restatement of
attention.mojo / the engine's append) on the first steps of the same schedule.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "llm-mojo_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "paged decode attn tokens/s + achieved HBM GB/s (% peak) at B=32, 1 GPU"
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E, AMD published


def _traffic_from_profiles():
    """HBM bytes per attention launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), from the committed summary."""
    path = os.path.join(REPO, "profiles", "attend_decode_cfg2_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def run_gpu(sched, data, steps, warmup, log):
    from pkv import LayerSpec, PagedKVCache, hip

    B = sched.B
    stream = hip.Stream()
    layers = [LayerSpec(sched.HQ, sched.HKV, sched.D, window=sched.WINDOW),
              LayerSpec(sched.HQ, sched.HKV, sched.D, window=0)]
    cache = PagedKVCache(layers, block_size=sched.BS, num_blocks=sched.num_blocks,
                         max_seqs=B, max_blocks_per_seq=sched.table_stride, max_q_len=1,
                         max_pos=sched.max_pos, scale=sched.SCALE, stream=stream)
    D = hip.DeviceArray.from_numpy
    # Initial state; data["pools"] stays pristine and is copied in before each run.
    fl = np.zeros(sched.num_blocks, np.int32)
    fl[:sched.free0.size] = sched.free0
    init = {"tables": D(sched.tables0), "lens": D(sched.lens0), "free": D(fl),
            "count": D(np.array([sched.free0.size], np.int32))}
    pristine = []
    for layer in range(2):
        for kv, pool in enumerate((cache.k_pools[layer], cache.v_pools[layer])):
            pristine.append((pool, data["pools"][layer][kv]))
    q, k_new, v_new = data["q"], data["k_new"], data["v_new"]
    pos = D(sched.pos)
    dec_off = D(sched.decode_tok_off())
    row_bytes = sched.kv_stride * 4
    ev = {}
    for j in sched.events:
        e = data["event_index"][j]
        ev[j] = dict(new_len=D(sched.retire_new_len(j)), pos=D(sched.admit_pos(j)),
                     off=D(sched.admit_tok_off(j)),
                     k=[data["admit_k"].ptr + (e * 2 + l) * sched.admit_rows * row_bytes
                        for l in range(2)],
                     v=[data["admit_v"].ptr + (e * 2 + l) * sched.admit_rows * row_bytes
                        for l in range(2)])
    outs = hip.DeviceArray((sched.STEPS, 2, B, 1, sched.HQ, sched.D), np.float32)
    scratch_out = hip.DeviceArray((2, B, 1, sched.HQ, sched.D), np.float32)
    qstep = B * sched.HQ * sched.D * 4
    kvstep = B * row_bytes
    st = stream.handle
    state = ((cache.tables, init["tables"]), (cache.table_lens, init["lens"]),
             (cache.free_list, init["free"]), (cache.free_count, init["count"]))

    def restore_state():
        # block-manager state back to the schedule's start (stream-ordered)
        for dst, src in state:
            hip.check(hip._lib().hipMemcpyAsync(dst.ptr, src.ptr, dst.nbytes,
                                                hip.hipMemcpyDeviceToDevice, st),
                      "hipMemcpyAsync")

    def step(i, events=None, first_pass=False):
        j = i % sched.STEPS
        if j in sched.events:
            e = ev[j]
            cache.rollback(e["new_len"].ptr)
            for layer in range(2):
                cache.append(layer, e["pos"].ptr, e["off"].ptr, e["k"][layer], e["v"][layer],
                             sched.ADMIT_CTX, sched.admit_rows)
        for layer in range(2):
            off = j * 2 + layer
            cache.append(layer, pos.ptr + j * B * 4, dec_off.ptr, k_new.ptr + off * kvstep,
                         v_new.ptr + off * kvstep, 1, B)
            out = (outs.ptr + off * qstep) if first_pass else (scratch_out.ptr + layer * qstep)
            if events is not None:
                events[i][layer][0].record(stream)
            cache.attend(layer, q.ptr + off * qstep, pos.ptr + j * B * 4, 1, out)
            if events is not None:
                events[i][layer][1].record(stream)

    def restore_all():
        for pool, src in pristine:
            pool.copy_from(src)
        restore_state()
        hip.synchronize()

    restore_all()
    log("pools in place")
    for i in range(warmup):
        if i > 0 and i % sched.STEPS == 0:
            restore_state()
        step(i)
    stream.synchronize()
    restore_all()
    log(f"warmup {warmup} steps done")

    def timed(events):
        # K steps bracketed by a device synchronisation and two events on the stream.
        t_start, t_stop = hip.Event(), hip.Event()
        hip.synchronize()
        t0 = time.perf_counter()
        t_start.record(stream)
        for i in range(steps):
            if i > 0 and i % sched.STEPS == 0:
                restore_state()  # part of the timed work
            step(i, events, first_pass=(events is None and i < sched.STEPS))
        t_stop.record(stream)
        t_stop.synchronize()
        hip.synchronize()
        return time.perf_counter() - t0, t_start.elapsed_ms(t_stop)

    # Pass 1 (the headline): nothing but the steps between the two events. Pass 2 (the
    # roofline): the same steps again from the same state, with an event pair around
    # every attention launch; an event record between launches idles the queue for a
    # few microseconds, which is why it is not in pass 1.
    wall, gpu_ms = timed(None)
    restore_all()
    fence_free = hip.hipEventDisableSystemFence
    evs = [[(hip.Event(fence_free), hip.Event(fence_free)) for _ in range(2)]
           for _ in range(steps)]
    _, gpu_ms_ev = timed(evs)
    log(f"timed {steps} steps: {gpu_ms:.2f} ms (with per-launch events {gpu_ms_ev:.2f} ms)")
    dur = np.zeros((steps, 2))
    nbytes = np.zeros((steps, 2))
    for i in range(steps):
        for layer in range(2):
            dur[i, layer] = evs[i][layer][0].elapsed_ms(evs[i][layer][1])
            nbytes[i, layer] = sched.attend_bytes(i % sched.STEPS, layer)
    status = cache.status.numpy()
    first_outs = outs.numpy()
    cache.free()
    return dict(wall_s=wall, gpu_ms=gpu_ms, gpu_ms_ev=gpu_ms_ev, dur_ms=dur, bytes=nbytes,
                outs=first_outs, status=status)


def run_cpu(sched, data, seconds, nthreads, log):
    """Reference CPU path (oracle) on the first steps of the same schedule: the engine's
    append and paged_attention_layer per sequence, head-pair tasks on `nthreads` threads
    (attention.mojo:276-287), sequences one after another (…batched.mojo:2951)."""
    from oracle import oracle as O

    B = sched.B
    st = O.CacheState(2, sched.kv_stride, sched.BS, sched.num_blocks, B, sched.table_stride,
                      alloc_pools=False)
    for layer in range(2):
        st.k_pools[layer] = data["pools"][layer][0].numpy().reshape(-1)
        st.v_pools[layer] = data["pools"][layer][1].numpy().reshape(-1)
    qh, kh, vh = data["q"].numpy(), data["k_new"].numpy(), data["v_new"].numpy()
    ak, av = data["admit_k"].numpy(), data["admit_v"].numpy()
    st.tables[:] = sched.tables0
    st.table_lens[:] = sched.lens0
    st.bm.free_list[:sched.free0.size] = sched.free0
    st.bm.count[0] = sched.free0.size
    log("cpu baseline inputs downloaded")
    outs = []
    elapsed = 0.0
    done = 0
    dec_off = sched.decode_tok_off()
    for j in range(sched.STEPS):
        t0 = time.perf_counter()
        if j in sched.events:
            e = data["event_index"][j]
            st.rollback(sched.retire_new_len(j))
            for layer in range(2):
                st.append(layer, sched.admit_pos(j), sched.admit_tok_off(j), ak[e, layer],
                          av[e, layer], sched.ADMIT_CTX)
        step_out = []
        for layer in range(2):
            st.append(layer, sched.pos[j], dec_off, kh[j, layer], vh[j, layer], 1)
            o = O.attend(qh[j, layer], st.k_pools[layer], st.v_pools[layer], st.tables,
                         st.table_lens, sched.pos[j], 1, sched.HQ, sched.HKV, sched.D, sched.BS,
                         sched.WINDOW if layer == 0 else 0, scale=sched.SCALE,
                         nthreads=nthreads, par=0)
            step_out.append(o)
        elapsed += time.perf_counter() - t0
        outs.append(step_out)
        done += 1
        if elapsed >= seconds:
            break
    log(f"cpu baseline: {done} steps in {elapsed:.1f}s on {nthreads} threads")
    return dict(steps=done, seconds=elapsed, outs=outs)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bound on the CPU-baseline sample (0 disables it)")
    ap.add_argument("--cpu-threads", type=int, default=8,
                    help="threads for the reference CPU path (8 = its Hq/2 head-pair tasks)")
    ap.add_argument("--quiet", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the paged KV path on one GPU only: every GPU box here has "
              "one GPU and this path has no multi-GPU leg (sharding is design-only, see "
              "DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2

    def log(msg):
        if not args.quiet:
            print(f"[bench] {msg}", file=sys.stderr, flush=True)

    from pkv import hip
    from pkv.workloads import DecodeSchedule

    if hip.device_count() < 1:
        print("bench.py needs a GPU: no HIP device visible", file=sys.stderr)
        return 1
    t = time.perf_counter()
    sched = DecodeSchedule(seed=args.seed)
    data = sched.device_data()
    hip.synchronize()
    log(f"config 2 built in {time.perf_counter() - t:.1f}s: {sched.num_blocks} blocks, "
        f"contexts {sched.ctx0.min()}..{sched.ctx0.max()}")
    g = run_gpu(sched, data, args.steps, args.warmup, log)
    steps = args.steps
    ms_per_step = g["gpu_ms"] / steps
    tok_s = sched.B * steps / (g["gpu_ms"] / 1e3)
    dur, nb = g["dur_ms"], g["bytes"]
    achieved = nb.sum() / (dur.sum() / 1e3) / 1e9
    glob_gbs = nb[:, 1].sum() / (dur[:, 1].sum() / 1e3) / 1e9
    slide_gbs = nb[:, 0].sum() / (dur[:, 0].sum() / 1e3) / 1e9
    traffic = _traffic_from_profiles()
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": traffic,
                "kernel": "stream_attend_kernel<256, float, 2> + stream_merge_kernel<256, double>",
                "avg_launch_us": round(dur.mean() * 1e3, 2),
                "algorithmic_bytes_per_launch": int(nb.mean())}
    result = {
        "metric": METRIC, "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded N(0,1) K/V/Q, seeded contexts U[128,8192], seeded "
                "random non-overlapping block tables",
        "config": {"workload": "BASELINE config 2: continuous-batching decode, 32 sequences, "
                               "sliding(1024)+global layers, 16q/8kv/256, block 16, fp32 KV, "
                               "retire 4 / admit 4 (256 tok) every 8 steps, 64-step schedule",
                   "batch": sched.B, "num_blocks": sched.num_blocks, "head_dim": sched.D,
                   "kv_heads": sched.HKV, "q_heads": sched.HQ, "block_size": sched.BS},
        "roofline": roofline,
        "attn_global_gbs": round(glob_gbs, 1),
        "attn_global_frac": round(glob_gbs / PEAK_HBM_GBS, 4),
        "attn_sliding_gbs": round(slide_gbs, 1),
        "attn_global_avg_us": round(dur[:, 1].mean() * 1e3, 2),
        "attn_sliding_avg_us": round(dur[:, 0].mean() * 1e3, 2),
        "ms_per_step_with_launch_events": round(g["gpu_ms_ev"] / steps, 4),
        "wall_s": round(g["wall_s"], 4),
        "append_status_ok": bool(np.all(g["status"] == 0)),
    }
    if args.cpu_seconds > 0:
        c = run_cpu(sched, data, args.cpu_seconds, args.cpu_threads, log)
        from oracle import oracle as O

        errs = [O.max_rel_err(g["outs"][j, layer], c["outs"][j][layer])
                for j in range(min(c["steps"], steps)) for layer in range(2)]
        result["cpu_baseline"] = {
            "value": round(sched.B * c["steps"] / c["seconds"], 2), "unit": "tokens/s",
            "cores": args.cpu_threads, "kind": "port",
            "sample": f"first {c['steps']} steps of the same 64-step schedule (both layers, "
                      f"appends + attention), reference-faithful: sequences in turn, "
                      f"{args.cpu_threads} head-pair tasks per call"}
        if errs:
            result["parity_sample_max_rel_err"] = float(f"{max(errs):.3g}")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
