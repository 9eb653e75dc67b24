#!/usr/bin/env python3
"""Paged decode benchmark on one MI355X: BASELINE.json config 2 through libpkv's C ABI.

One step = one continuous-batching decode step of 32 sequences on a sliding-window
(1024) and a global layer (16 q / 8 kv heads, head_dim 256, block 16, fp32 pools):
per layer one pkv_append_attend call: the K/V append (one token per sequence, into
partially filled blocks) and split-K paged attention, whose launch also writes the appended
rows; every 8th step first retires 4 sequences (their blocks go
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
PEAK_FP64_MFMA_TFLOPS = 78.6  # MI355X dense fp64 matrix, AMD published
PEAK_BF16_MFMA_TFLOPS = 2500.0  # MI355X dense bf16 matrix, AMD published


def _profile_figures(name):
    """The figures a committed rocprofv3 summary under profiles/ records as `key: value`
    lines: bytes_per_launch (HBM bytes per launch from --pmc FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration) and algorithmic_bytes_per_launch (this script's
    figure for the same launches of the same run)."""
    out = {}
    try:
        with open(os.path.join(REPO, "profiles", name)) as f:
            for line in f:
                k, sep, v = line.partition(":")
                if sep and k in ("bytes_per_launch", "algorithmic_bytes_per_launch"):
                    out[k] = int(v.strip().replace(",", ""))
    except (OSError, ValueError):
        pass
    return out


def _set_traffic(roof, name):
    """roofline.traffic: the measured HBM bytes per launch of the profiled run, carried to
    this run's launches through their ratio to the algorithmic bytes of the same profiled
    launches (both from one window; with the window the profile used, the measured figure
    itself)."""
    fig = _profile_figures(name)
    meas, alg = fig.get("bytes_per_launch"), fig.get("algorithmic_bytes_per_launch")
    if meas is None:
        roof["traffic"] = None
        return roof
    if alg:
        ratio = meas / alg
        roof["traffic"] = int(round(ratio * roof["algorithmic_bytes_per_launch"]))
        roof["traffic_vs_algorithmic"] = round(ratio, 4)
    else:
        roof["traffic"] = meas
    roof["traffic_profile"] = "profiles/" + name
    return roof


def run_gpu(sched, data, steps, warmup, log):
    from pkv import LayerSpec, PagedKVCache, hip

    B = sched.B
    stream = hip.Stream()
    L = sched.L
    layers = [LayerSpec(sched.HQ, sched.HKV, sched.D, window=w) for w in sched.windows]
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
    for layer in range(L):
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
                     k=[data["admit_k"].ptr + (e * L + l) * sched.admit_rows * row_bytes
                        for l in range(L)],
                     v=[data["admit_v"].ptr + (e * L + l) * sched.admit_rows * row_bytes
                        for l in range(L)])
    outs = hip.DeviceArray((sched.STEPS, L, B, 1, sched.HQ, sched.D), np.float32)
    scratch_out = hip.DeviceArray((L, B, 1, sched.HQ, sched.D), np.float32)
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
            for layer in range(L):
                cache.append(layer, e["pos"].ptr, e["off"].ptr, e["k"][layer], e["v"][layer],
                             sched.ADMIT_CTX, sched.admit_rows)
        for layer in range(L):
            off = j * L + layer
            out = (outs.ptr + off * qstep) if first_pass else (scratch_out.ptr + layer * qstep)
            if events is None:
                # the step as an engine runs it: append + attention in one call, whose
                # attention launch also writes the appended rows (pkv_append_attend)
                cache.append_attend(layer, pos.ptr + j * B * 4, dec_off.ptr,
                                    k_new.ptr + off * kvstep, v_new.ptr + off * kvstep, 1, B,
                                    q.ptr + off * qstep, 1, out)
                continue
            # roofline pass: the append as its own call, the event pair around the attention
            cache.append(layer, pos.ptr + j * B * 4, dec_off.ptr, k_new.ptr + off * kvstep,
                         v_new.ptr + off * kvstep, 1, B)
            events[i][layer][0].record(stream)
            cache.attend(layer, q.ptr + off * qstep, pos.ptr + j * B * 4, 1, out)
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
    evs = [[(hip.Event(fence_free), hip.Event(fence_free)) for _ in range(L)]
           for _ in range(steps)]
    _, gpu_ms_ev = timed(evs)
    log(f"timed {steps} steps: {gpu_ms:.2f} ms (with per-launch events {gpu_ms_ev:.2f} ms)")
    dur = np.zeros((steps, L))
    nbytes = np.zeros((steps, L))
    for i in range(steps):
        for layer in range(L):
            dur[i, layer] = evs[i][layer][0].elapsed_ms(evs[i][layer][1])
            nbytes[i, layer] = sched.attend_bytes(i % sched.STEPS, layer)
    status = cache.status.numpy()
    first_outs = outs.numpy()
    cache.free()
    return dict(wall_s=wall, gpu_ms=gpu_ms, gpu_ms_ev=gpu_ms_ev, dur_ms=dur, bytes=nbytes,
                outs=first_outs, status=status)


def host_cpu_info():
    """The GPU box host's CPU as the baseline record states it: model name, logical CPUs
    (os.cpu_count / nproc), physical cores (distinct (socket, core) pairs of
    /proc/cpuinfo, as lscpu counts them) and the OpenMP thread share of this job."""
    model, cores = None, set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    return {"model": model, "logical_cpus": os.cpu_count(),
            "physical_cores": len(cores) or None,
            "omp_num_threads": int(omp) if omp and omp.isdigit() else None}


def run_cpu(sched, data, seconds, nthreads, log, par=0):
    """Reference CPU path (oracle) on the steps of the same schedule, up to `seconds` of
    work: the engine's append and paged_attention_layer per sequence. par 0 is the
    reference's own dispatch: head-pair tasks on `nthreads` threads (attention.mojo:276-287),
    sequences one after another (…batched.mojo:2951). par 3 is the all-cores batched mode:
    every (sequence, head pair) task of a step on `nthreads` threads at once."""
    from oracle import oracle as O
    O.use_host_build()

    B, L = sched.B, sched.L
    st = O.CacheState(L, sched.kv_stride, sched.BS, sched.num_blocks, B, sched.table_stride,
                      alloc_pools=False)
    for layer in range(L):
        st.k_pools[layer] = data["pools"][layer][0].numpy().reshape(-1)
        st.v_pools[layer] = data["pools"][layer][1].numpy().reshape(-1)
    qh, kh, vh = data["q"].numpy(), data["k_new"].numpy(), data["v_new"].numpy()
    ak, av = data["admit_k"].numpy(), data["admit_v"].numpy()
    st.tables[:] = sched.tables0
    st.table_lens[:] = sched.lens0
    st.bm.free_list[:sched.free0.size] = sched.free0
    st.bm.count[0] = sched.free0.size
    log("cpu baseline inputs downloaded")
    outs, exact = [], []
    elapsed = 0.0
    done = 0
    dec_off = sched.decode_tok_off()
    for j in range(sched.STEPS):
        t0 = time.perf_counter()
        if j in sched.events:
            e = data["event_index"][j]
            st.rollback(sched.retire_new_len(j))
            for layer in range(L):
                st.append(layer, sched.admit_pos(j), sched.admit_tok_off(j), ak[e, layer],
                          av[e, layer], sched.ADMIT_CTX)
        step_out = []
        for layer in range(L):
            st.append(layer, sched.pos[j], dec_off, kh[j, layer], vh[j, layer], 1)
            o = O.attend(qh[j, layer], st.k_pools[layer], st.v_pools[layer], st.tables,
                         st.table_lens, sched.pos[j], 1, sched.HQ, sched.HKV, sched.D, sched.BS,
                         sched.windows[layer], scale=sched.SCALE,
                         nthreads=nthreads, par=par)
            step_out.append(o)
        elapsed += time.perf_counter() - t0
        if j < 2 and par == 0:  # float64 attention of the same inputs (outside the sample)
            for layer in range(L):
                exact.append((j, layer, O.attend_f64(
                    qh[j, layer], st.k_pools[layer], st.v_pools[layer], st.tables,
                    sched.pos[j], 1, sched.HQ, sched.HKV, sched.D, sched.BS,
                    sched.windows[layer], scale=sched.SCALE)))
        outs.append(step_out)
        done += 1
        if elapsed >= seconds:
            break
    log(f"cpu baseline (par {par}): {done} steps in {elapsed:.1f}s on {nthreads} threads")
    return dict(steps=done, seconds=elapsed, outs=outs, exact=exact)


class _Setup:
    """A PagedKVCache for workload `w` in its initial block-manager state, the pools
    copied from the workload's device data, and a stream-ordered restore of the state."""

    def __init__(self, w, layers, kv_dtype, q_len, stream):
        from pkv import LayerSpec, PagedKVCache, hip

        self.hip = hip
        self.stream = stream
        specs = [LayerSpec(w.HQ, w.HKV, w.D, window=w.WINDOW, kv_dtype=kv_dtype)
                 for _ in range(layers)]
        self.cache = PagedKVCache(specs, block_size=w.BS, num_blocks=w.num_blocks,
                                  max_seqs=w.B, max_blocks_per_seq=w.table_stride,
                                  max_q_len=q_len, max_pos=w.max_pos, scale=w.SCALE,
                                  stream=stream)
        D = hip.DeviceArray.from_numpy
        tables = np.zeros((w.B, w.table_stride), np.int32)
        tables[:, :w.tables0.shape[1]] = w.tables0
        fl = np.zeros(w.num_blocks, np.int32)
        fl[:w.free0.size] = w.free0
        c = self.cache
        self.pairs = ((c.tables, D(tables)), (c.table_lens, D(np.asarray(w.lens0, np.int32))),
                      (c.free_list, D(fl)), (c.free_count, D(np.array([w.free0.size], np.int32))))
        self.restore()
        hip.synchronize()

    def restore(self):
        h = self.hip
        for dst, src in self.pairs:
            h.check(h._lib().hipMemcpyAsync(dst.ptr, src.ptr, dst.nbytes, h.hipMemcpyDeviceToDevice,
                                            self.stream.handle), "hipMemcpyAsync")


def _timed(hip, stream, steps, body):
    """Runs body(i) for i < steps between two events on `stream`; returns milliseconds."""
    t0, t1 = hip.Event(), hip.Event()
    hip.synchronize()
    t0.record(stream)
    for i in range(steps):
        body(i)
    t1.record(stream)
    t1.synchronize()
    return t0.elapsed_ms(t1)


def _event_pairs(hip, n):
    f = hip.hipEventDisableSystemFence
    return [(hip.Event(f), hip.Event(f)) for _ in range(n)]


def _line(metric, value, unit, steps, warmup, ms_per_step, dtype, workload, roofline, extra):
    r = {"metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": steps,
         "warmup": warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
         "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic: seeded "
         "N(0,1) K/V/Q, seeded random non-overlapping block tables",
         "config": {"workload": workload}, "roofline": roofline}
    r.update(extra)
    if "data" in extra:
        r["data"] = extra["data"]
    return r


def _roofline(nbytes, dur_ms, kernel, flops=None):
    achieved = nbytes / (dur_ms / 1e3) / 1e9
    r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
         "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None, "kernel": kernel,
         "avg_launch_us": round(dur_ms * 1e3, 2), "algorithmic_bytes_per_launch": int(nbytes)}
    if flops is not None:  # the fp32-pool verify runs its dot products on the fp64 MFMA
        tf = flops / (dur_ms / 1e3) / 1e12
        r["fp64_mfma_tflops"] = round(tf, 2)
        r["fp64_mfma_frac"] = round(tf / PEAK_FP64_MFMA_TFLOPS, 4)
    return r


def bench_config1(args, log):
    """Config 1: one sequence, append at 512 (new block) + attend 513 keys, fp32. A step
    ends with a rollback to 512 tokens, which returns the block to the back of the free
    list, so every step starts from the same state."""
    from pkv import F32, hip
    from pkv.workloads import SingleStep

    w = SingleStep(seed=args.seed)
    d = w.device_data()
    stream = hip.Stream()
    S = _Setup(w, 1, F32, 1, stream)
    c = S.cache
    c.k_pools[0].copy_from(d["k"])
    c.v_pools[0].copy_from(d["v"])
    D = hip.DeviceArray.from_numpy
    dpos, doff, dnl = D(w.pos), D(np.array([0, 1], np.int32)), D(w.pos)
    out = hip.DeviceArray((1, 1, w.HQ, w.D), np.float32)
    ev = _event_pairs(hip, args.steps)

    def step(i, events=None):
        c.append(0, dpos.ptr, doff.ptr, d["k_new"], d["v_new"], 1, 1, batch=1)
        if events:
            events[i][0].record(stream)
        c.attend(0, d["q"], dpos.ptr, 1, out, batch=1)
        if events:
            events[i][1].record(stream)
        c.rollback(dnl.ptr, batch=1)

    for i in range(args.warmup):
        step(i)
    ms = _timed(hip, stream, args.steps, step)
    _timed(hip, stream, args.steps, lambda i: step(i, ev))
    dur = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    got = out.numpy()
    res = _line("config 1 single-sequence decode step (append + attend 513 keys) latency",
                1e3 / ms * args.steps, "steps/s", args.steps, args.warmup, ms / args.steps,
                "f32", "BASELINE config 1: 1 sequence, ctx 512 -> append at 512 into a new "
                "block, attend 513 keys, 16q/8kv/256, block 16, 256-block pool, fp32",
                _roofline(w.attend_bytes(), dur, "stream_attend_kernel<256, float, 2>"),
                {"attend_us": round(dur * 1e3, 2)})
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        O.use_host_build()

        st = O.CacheState(1, w.kv_stride, w.BS, w.num_blocks, 1, w.table_stride,
                          alloc_pools=False)
        st.k_pools[0] = d["k"].numpy().reshape(-1).copy()
        st.v_pools[0] = d["v"].numpy().reshape(-1).copy()
        kn, vn, q = d["k_new"].numpy(), d["v_new"].numpy(), d["q"].numpy()
        n, el, ref = 0, 0.0, None
        while el < args.cpu_seconds and n < 1000:
            st.tables[:, :w.tables0.shape[1]] = w.tables0
            st.table_lens[:] = w.lens0
            st.bm.free_list[:w.free0.size] = w.free0
            st.bm.count[0] = w.free0.size
            t = time.perf_counter()
            st.append(0, w.pos, [0, 1], kn, vn, 1)
            ref = O.attend(q, st.k_pools[0], st.v_pools[0], st.tables, st.table_lens, w.pos, 1,
                           w.HQ, w.HKV, w.D, w.BS, 0, scale=w.SCALE, nthreads=args.cpu_threads)
            el += time.perf_counter() - t
            n += 1
        res["cpu_baseline"] = {"value": round(n / el, 2), "unit": "steps/s",
                               "cores": args.cpu_threads, "kind": "port", "host": host_cpu_info(),
                               "sample": f"{n} steps (append + paged_attention_layer, "
                                         f"{args.cpu_threads} head-pair tasks)"}
        res["parity_sample_max_rel_err"] = float(f"{O.max_rel_err(got, ref):.3g}")
    return res


def bench_config3(args, log):
    """Config 3: 8 sequences x 32768 keys over bf16 pages; a step appends the token at
    position 32767 (no allocation: the slot is in the last table block) and attends."""
    from pkv import BF16, hip
    from pkv.workloads import LongDecode

    w = LongDecode(seed=args.seed)
    d = w.device_data()
    stream = hip.Stream()
    S = _Setup(w, 1, BF16, 1, stream)
    c = S.cache
    c.k_pools[0].copy_from(d["k"])
    c.v_pools[0].copy_from(d["v"])
    D = hip.DeviceArray.from_numpy
    dpos, doff = D(w.pos), D(np.arange(w.B + 1, dtype=np.int32))
    out = hip.DeviceArray((w.B, 1, w.HQ, w.D), np.float32)
    ev = _event_pairs(hip, args.steps)

    def step(i, events=None):
        c.append(0, dpos.ptr, doff.ptr, d["k_new"], d["v_new"], 1, w.B)
        if events:
            events[i][0].record(stream)
        c.attend(0, d["q"], dpos.ptr, 1, out)
        if events:
            events[i][1].record(stream)

    for i in range(args.warmup):
        step(i)
    ms = _timed(hip, stream, args.steps, step)
    _timed(hip, stream, args.steps, lambda i: step(i, ev))
    dur = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    got = out.numpy()
    res = _line("config 3 long-context paged decode tokens/s (B=8, 32K keys, bf16 pages)",
                w.B * args.steps / (ms / 1e3), "tokens/s", args.steps, args.warmup,
                ms / args.steps, "bf16",
                "BASELINE config 3: 8 sequences x 32768 keys, 16q/8kv/256, block 16, "
                "16384-block pool, bf16 K/V, fp32 Q, append + attend",
                _roofline(w.attend_bytes(), dur,
                          "stream_attend_kernel<256, bf16, 2> + stream_merge_kernel<256, float>"),
                {"attend_us": round(dur * 1e3, 2)})
    _set_traffic(res["roofline"], "stream_attend_bf16_cfg3_traffic.md")
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        O.use_host_build()

        k, v, q = d["k"].numpy().reshape(-1), d["v"].numpy().reshape(-1), d["q"].numpy()
        tables = np.ascontiguousarray(w.tables0)
        n, el, ref = 0, 0.0, None
        while el < args.cpu_seconds and n < 100:
            t = time.perf_counter()
            ref = O.attend(q, k, v, tables, w.lens0, w.pos, 1, w.HQ, w.HKV, w.D, w.BS, 0,
                           scale=w.SCALE, nthreads=args.cpu_threads)
            el += time.perf_counter() - t
            n += 1
        res["cpu_baseline"] = {"value": round(w.B * n / el, 3), "unit": "tokens/s",
                               "cores": args.cpu_threads, "kind": "port", "host": host_cpu_info(),
                               "sample": f"{n} attention steps (8 sequences in turn, "
                                         f"{args.cpu_threads} head-pair tasks per call; the "
                                         f"pre-append pools, so the 32768th key differs)"}
        log("config 3 cpu sample done")
    return res


def bench_config4(args, log):
    """Config 4: chunked prefill. A step appends the 4 x 2048-token chunks into fresh
    blocks and runs the MFMA prefill attention; a rollback to the prefix lengths returns
    the chunk's blocks so every step starts from the same state."""
    from pkv import BF16, hip
    from pkv.workloads import PrefillChunk

    w = PrefillChunk(seed=args.seed)
    d = w.device_data()
    stream = hip.Stream()
    S = _Setup(w, 1, BF16, 1, stream)
    c = S.cache
    c.k_pools[0].copy_from(d["k"])
    c.v_pools[0].copy_from(d["v"])
    D = hip.DeviceArray.from_numpy
    dpos, doff = D(w.pos), D(w.tok_off())
    dnl = D(w.prefix.astype(np.int32))
    out = hip.DeviceArray((w.rows, w.HQ, w.D), np.float32)
    ev = _event_pairs(hip, args.steps)

    def step(i, events=None):
        c.append(0, dpos.ptr, doff.ptr, d["k_new"], d["v_new"], w.CHUNK, w.rows)
        if events:
            events[i][0].record(stream)
        c.prefill(0, d["q"], dpos.ptr, doff.ptr, w.CHUNK, out)
        if events:
            events[i][1].record(stream)
        c.rollback(dnl.ptr)

    for i in range(args.warmup):
        step(i)
    ms = _timed(hip, stream, args.steps, step)
    _timed(hip, stream, args.steps, lambda i: step(i, ev))
    dur = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    got = out.numpy()
    flops = w.flops()
    tf = flops / (dur / 1e3) / 1e12
    roof = {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK_BF16_MFMA_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / PEAK_BF16_MFMA_TFLOPS, 4), "traffic": None,
            "kernel": "prefill_kernel<2>", "avg_launch_us": round(dur * 1e3, 2),
            "algorithmic_flops_per_launch": int(flops),
            "note": "algorithmic flops (QK^T + PV, causal); the kernel issues 1.5x that on "
                    "MFMA (PV runs twice, P split into bf16 hi + lo)"}
    res = _line("config 4 chunked prefill query tokens/s (4 x 2048-token chunks, bf16, MFMA)",
                w.rows * args.steps / (ms / 1e3), "tokens/s", args.steps, args.warmup,
                ms / args.steps, "bf16",
                "BASELINE config 4: 4 sequences, prefix U[0,6144], 2048-token chunk appended "
                "into fresh blocks, causal attention over prefix + chunk, 16q/8kv/256, block "
                "16, bf16 Q/K/V, fp32 accumulation", roof,
                {"prefill_us": round(dur * 1e3, 2), "prefixes": w.prefix.tolist()})
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        O.use_host_build()

        k, v = d["k"].numpy().reshape(-1), d["v"].numpy().reshape(-1)
        kn = d["k_new"].numpy().reshape(-1, w.kv_stride)
        vn = d["v_new"].numpy().reshape(-1, w.kv_stride)
        q32 = O.bf16_to_f32(d["q"].numpy().reshape(w.rows, w.HQ, w.D))
        st = O.CacheState(1, w.kv_stride, w.BS, w.num_blocks, w.B, w.table_stride,
                          dtype=np.uint16, alloc_pools=False)
        st.k_pools[0], st.v_pools[0] = k, v
        st.tables[:, :w.tables0.shape[1]] = w.tables0
        st.table_lens[:] = w.lens0
        st.bm.free_list[:w.free0.size] = w.free0
        st.bm.count[0] = w.free0.size
        st.append(0, w.pos, w.tok_off(), kn, vn, w.CHUNK)
        # The reference prefills token by token; sample the first n queries of sequence 0
        # (each one paged_attention_layer call on the head-pair threads) within the bound.
        n, el, errs = 0, 0.0, []
        while el < args.cpu_seconds and n < w.CHUNK:
            t = time.perf_counter()
            ref = O.attend(q32[n:n + 1].reshape(1, 1, w.HQ, w.D), st.k_pools[0], st.v_pools[0],
                           st.tables[:1], st.table_lens[:1], w.pos[:1] + n, 1, w.HQ, w.HKV,
                           w.D, w.BS, 0, scale=w.SCALE, nthreads=args.cpu_threads)
            el += time.perf_counter() - t
            errs.append(O.max_rel_err(got[n], ref[0, 0]))
            n += 1
        res["cpu_baseline"] = {"value": round(n / el, 2), "unit": "tokens/s",
                               "cores": args.cpu_threads, "kind": "port", "host": host_cpu_info(),
                               "sample": f"first {n} chunk queries of sequence 0 (prefix "
                                         f"{int(w.prefix[0])}), one paged_attention_layer call "
                                         f"each, {args.cpu_threads} head-pair tasks"}
        res["parity_sample_max_rel_err"] = float(f"{max(errs):.3g}")
    return res


VERIFY_BF16_KERNEL = "stream_bf16_mfma_kernel<paged> (bf16 MFMA) + stream_merge_kernel<256, float>"


def bench_config5(args, log):
    """Config 5: per iteration, MTP reads (4 draft steps x 2 layers, read-only at pos-1),
    4-token verify append + causal attention on both layers, rollback to the accepted
    length; the 32-iteration schedule repeats with the block-manager state restored."""
    from pkv import BF16, F32, hip
    from pkv.workloads import VerifySchedule

    bf16 = args.kv_dtype == "bf16"
    w = VerifySchedule(seed=args.seed, bf16=bf16)
    d = w.device_data()
    stream = hip.Stream()
    L, B, DR = w.LAYERS, w.B, w.DRAFT
    S = _Setup(w, L, BF16 if bf16 else F32, DR, stream)
    c = S.cache
    for layer in range(L):
        c.k_pools[layer].copy_from(d["pools"][layer][0])
        c.v_pools[layer].copy_from(d["pools"][layer][1])
    pristine = [(c.k_pools[l], d["pools"][l][0]) for l in range(L)] + \
               [(c.v_pools[l], d["pools"][l][1]) for l in range(L)]
    D = hip.DeviceArray.from_numpy
    dpos = [D(w.pos(it)) for it in range(w.ITERS)]
    dpm1 = [D(w.pos(it) - 1) for it in range(w.ITERS)]
    dnl = [D(w.new_len(it)) for it in range(w.ITERS)]
    doff = D(w.tok_off())
    out_v = hip.DeviceArray((w.ITERS, L, B, DR, w.HQ, w.D), np.float32)
    out_m = hip.DeviceArray((B, 1, w.HQ, w.D), np.float32)
    qstep, mstep = B * DR * w.HQ * w.D * 4, B * w.HQ * w.D * 4
    kvstep = B * DR * w.kv_stride * w.elt
    ev = [_event_pairs(hip, L) for _ in range(args.steps)]

    def iteration(i, events=None):
        it = i % w.ITERS
        if i > 0 and it == 0:
            S.restore()
        for dstep in range(DR):
            for layer in range(L):
                c.attend(layer, d["mtp_q"].ptr + ((it * L + layer) * DR + dstep) * mstep,
                         dpm1[it].ptr, 1, out_m)
        for layer in range(L):
            n = it * L + layer
            c.append(layer, dpos[it].ptr, doff.ptr, d["k_new"].ptr + n * kvstep,
                     d["v_new"].ptr + n * kvstep, DR, B * DR)
        for layer in range(L):
            n = it * L + layer
            if events:
                events[i][layer][0].record(stream)
            c.attend(layer, d["q"].ptr + n * qstep, dpos[it].ptr, DR, out_v.ptr + n * qstep)
            if events:
                events[i][layer][1].record(stream)
        c.rollback(dnl[it].ptr)

    def reset():
        for pool, src in pristine:
            pool.copy_from(src)
        S.restore()
        hip.synchronize()

    for i in range(args.warmup):
        iteration(i)
    reset()
    ms = _timed(hip, stream, args.steps, iteration)
    got = out_v.numpy()
    reset()
    _timed(hip, stream, args.steps, lambda i: iteration(i, ev))
    dur = np.array([[a.elapsed_ms(b) for a, b in e] for e in ev])
    its = [i % w.ITERS for i in range(args.steps)]
    nbytes = float(np.mean([w.verify_bytes(it) for it in its]))
    flops = float(np.mean([w.verify_flops(it) for it in its]))
    if bf16:
        res = _line("config 5 bf16-pool variant: MTP verify query tokens/s (16 seq, draft 4, 2 "
                    "layers, shared KV, rollback)", B * DR * args.steps / (ms / 1e3), "tokens/s",
                    args.steps, args.warmup, ms / args.steps, "bf16",
                    "config 5's schedule with bf16 K/V pools (fp32 Q): 16 sequences, ctx "
                    "U[512,4096], 2 global layers 16q/8kv/256, block 16; per iteration 4 MTP "
                    "reads at pos-1 per layer, 4-token verify append + causal attention, accept "
                    "U{0..4}, rollback; 32-iteration schedule",
                    _roofline(nbytes, float(dur.mean()), VERIFY_BF16_KERNEL),
                    {"verify_attend_us": round(float(dur.mean()) * 1e3, 2)})
        _set_traffic(res["roofline"], "verify_mtp_bf16_traffic.md")
    else:
        res = _line("config 5 MTP verify query tokens/s (16 seq, draft 4, 2 layers, shared KV, "
                    "rollback)", B * DR * args.steps / (ms / 1e3), "tokens/s", args.steps,
                    args.warmup, ms / args.steps, "f32",
                    "BASELINE config 5: 16 sequences, ctx U[512,4096], 2 global layers 16q/8kv/256 "
                    "fp32, block 16; per iteration 4 MTP reads at pos-1 per layer, 4-token verify "
                    "append + causal attention, accept U{0..4}, rollback; 32-iteration schedule",
                    _roofline(nbytes, float(dur.mean()), "stream_mfma_kernel<256, 2, 1, 1, paged> "
                              "(fp64 MFMA) + stream_merge_kernel<256, double>", flops=flops),
                    {"verify_attend_us": round(float(dur.mean()) * 1e3, 2)})
        _set_traffic(res["roofline"], "verify_mtp_cfg5_traffic.md")
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        O.use_host_build()

        st = O.CacheState(L, w.kv_stride, w.BS, w.num_blocks, B, w.table_stride,
                          alloc_pools=False, dtype=np.uint16 if bf16 else np.float32)
        for layer in range(L):
            st.k_pools[layer] = d["pools"][layer][0].numpy().reshape(-1).copy()
            st.v_pools[layer] = d["pools"][layer][1].numpy().reshape(-1).copy()
        st.tables[:, :w.tables0.shape[1]] = w.tables0
        st.table_lens[:] = w.lens0
        st.bm.free_list[:w.free0.size] = w.free0
        st.bm.count[0] = w.free0.size
        qa, ma = d["q"].numpy(), d["mtp_q"].numpy()
        kn, vn = d["k_new"].numpy(), d["v_new"].numpy()
        n, el, errs, e64, own = 0, 0.0, [], [], []
        for it in range(w.ITERS):
            t = time.perf_counter()
            pos = w.pos(it)
            for dstep in range(DR):
                for layer in range(L):
                    O.attend(ma[it * L + layer, dstep], st.k_pools[layer], st.v_pools[layer],
                             st.tables, st.table_lens, pos - 1, 1, w.HQ, w.HKV, w.D, w.BS, 0,
                             scale=w.SCALE, nthreads=args.cpu_threads)
            for layer in range(L):
                st.append(layer, pos, w.tok_off(), kn[it * L + layer], vn[it * L + layer], DR)
            refs = []
            for layer in range(L):
                ref = O.attend(qa[it * L + layer], st.k_pools[layer], st.v_pools[layer],
                               st.tables, st.table_lens, pos, DR, w.HQ, w.HKV, w.D, w.BS, 0,
                               scale=w.SCALE, nthreads=args.cpu_threads)
                if it < args.steps:  # iterations the timed pass wrote
                    errs.append(O.max_rel_err(got[it, layer], ref))
                refs.append(ref)
            el += time.perf_counter() - t
            if it == 0 and not bf16:  # float64 attention of iteration 0 (outside the sample)
                for layer in range(L):
                    ex = O.attend_f64(qa[layer], st.k_pools[layer], st.v_pools[layer],
                                      st.tables, pos, DR, w.HQ, w.HKV, w.D, w.BS, 0,
                                      scale=w.SCALE)
                    e64.append(O.max_rel_err(got[0, layer], ex))
                    own.append(O.max_rel_err(refs[layer], ex))
            t = time.perf_counter()
            st.rollback(w.new_len(it))
            el += time.perf_counter() - t
            n += 1
            if el >= args.cpu_seconds:
                break
        res["cpu_baseline"] = {"value": round(B * DR * n / el, 2), "unit": "tokens/s",
                               "cores": args.cpu_threads, "kind": "port", "host": host_cpu_info(),
                               "sample": f"first {n} iterations of the schedule (MTP reads, "
                                         f"appends, verify as {DR} sequential "
                                         f"paged_attention_layer calls per sequence, rollback)"}
        res["parity_sample_max_rel_err"] = float(f"{max(errs):.3g}")
        res["parity_sample"] = {"iterations": min(n, args.steps),
                                "max_rel_err_vs_cpu_fp32": float(f"{max(errs):.3g}")}
        if e64:
            res["parity_sample"].update({"max_rel_err_vs_float64": float(f"{max(e64):.3g}"),
                                         "cpu_fp32_vs_float64": float(f"{max(own):.3g}"),
                                         "float64_iterations": 1})
        else:
            res["parity_sample"]["bound"] = "2e-2 (bf16 pools; the reference path on the same bf16 values)"
    return res


def bench_producer(args, log):
    """The producer step fused with the append (pkv_append_qkv: per-head rms_norm of Q / K,
    rms_norm_noscale of V, RoPE, K/V rows into the pages) at config 4's prefill shape
    (4 x 2048 tokens, bf16 pools, bf16 Q out; the timed `value`) and config 2's decode shape
    (32 tokens, fp32 pools and Q). Every table already covers its positions, so a step
    rewrites the same rows and the allocation pops nothing."""
    from pkv import BF16, F32, LayerSpec, PagedKVCache, hip, synth

    HQ, HKV, D, BS = 16, 8, 256, 16
    stream = hip.Stream()

    def shape_leg(B, ntok, pos0, kv_dtype, q_dtype, steps, warmup, seed):
        span = (int(pos0.max()) + ntok) // BS + 1
        cache = PagedKVCache([LayerSpec(HQ, HKV, D, kv_dtype=kv_dtype)], block_size=BS,
                             num_blocks=B * span, max_seqs=B, max_blocks_per_seq=span,
                             stream=stream)
        cache.tables.upload(np.arange(B * span, dtype=np.int32).reshape(B, span))
        cache.table_lens.upload(np.full(B, span, np.int32))
        cache.free_count.upload(np.zeros(1, np.int32))
        rows = B * ntok
        q = synth.normal((rows, HQ * D), seed)
        k = synth.normal((rows, HKV * D), seed + 1)
        v = synth.normal((rows, HKV * D), seed + 2)
        qw = synth.normal((D,), seed + 3)
        kw = synth.normal((D,), seed + 4)
        q_out = hip.DeviceArray((rows, HQ * D), np.uint16 if q_dtype == BF16 else np.float32)
        D_ = hip.DeviceArray.from_numpy
        dpos = D_(pos0.astype(np.int32))
        doff = D_((np.arange(B + 1) * ntok).astype(np.int32))
        ev = _event_pairs(hip, steps)

        def step(i, events=None):
            if events:
                events[i][0].record(stream)
            cache.append_qkv(0, dpos.ptr, doff.ptr, q, k, v, qw, kw, q_out, ntok, rows, False,
                             q_dtype)
            if events:
                events[i][1].record(stream)

        for i in range(warmup):
            step(i)
        ms = _timed(hip, stream, steps, step)
        _timed(hip, stream, steps, lambda i: step(i, ev))
        dur = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
        st_ok = bool(np.all(cache.status.numpy() == 0))
        elt = 2 if kv_dtype == BF16 else 4
        qelt = 2 if q_dtype == BF16 else 4
        # read Q/K/V rows (fp32) + 2 weights; write Q out + K/V pool rows; table entries
        nbytes = rows * ((HQ + 2 * HKV) * D * 4 + HQ * D * qelt + 2 * HKV * D * elt + 4) + 2 * D * 4
        arrays = dict(q=q, k=k, v=v, qw=qw, kw=kw, q_out=q_out, pos=pos0, cache=cache)
        return ms, dur, nbytes, st_ok, arrays

    rng = np.random.default_rng(args.seed)
    prefix = rng.integers(0, 6145, 4)
    pf_ms, pf_dur, pf_bytes, pf_ok, _ = shape_leg(4, 2048, prefix, BF16, BF16, args.steps,
                                                  args.warmup, 101)
    dec_pos = rng.integers(128, 8193, 32)
    dc_ms, dc_dur, dc_bytes, dc_ok, dec = shape_leg(32, 1, dec_pos, F32, F32, args.steps,
                                                    args.warmup, 201)
    roof = _roofline(pf_bytes, pf_dur, "alloc_kernel + qkv_append_kernel<256, 2>")
    _set_traffic(roof, "producer_qkv_append_traffic.md")
    res = _line("producer step (rms_norm + RoPE + KV append) tokens/s, 4 x 2048-token prefill "
                "chunks", 4 * 2048 * args.steps / (pf_ms / 1e3), "tokens/s", args.steps,
                args.warmup, pf_ms / args.steps, "f32 in, bf16 out",
                "pkv_append_qkv at BASELINE config 4's shape: 4 sequences x 2048 tokens at "
                "prefixes U[0,6144], 16q/8kv/256, block 16, fp32 projections in, bf16 pools "
                "and bf16 Q out, sliding-layer RoPE", roof,
                {"status_ok": pf_ok and dc_ok,
                 "decode_shape": {"tokens": 32, "us_per_call": round(dc_dur * 1e3, 2),
                                  "ms_per_step_back_to_back": round(dc_ms / args.steps, 4),
                                  "gbs": round(dc_bytes / (dc_dur / 1e3) / 1e9, 1),
                                  "bytes_per_call": int(dc_bytes),
                                  "pools": "fp32"}})
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        O.use_host_build()

        c = dec["cache"]
        q, k, v = dec["q"].numpy(), dec["k"].numpy(), dec["v"].numpy()
        qw, kw = dec["qw"].numpy(), dec["kw"].numpy()
        got_q = dec["q_out"].numpy()
        st = O.CacheState(1, HKV * D, BS, c.num_blocks, 32, c.table_stride)
        st.tables[:] = np.arange(32 * c.table_stride, dtype=np.int32).reshape(32, -1)
        st.table_lens[:] = c.table_stride
        st.bm.count[0] = 0
        off = (np.arange(33)).astype(np.int32)
        n, el, want_q = 0, 0.0, None
        while el < args.cpu_seconds and n < 2000:
            t = time.perf_counter()
            _, want_q = O.append_qkv(st, 0, dec["pos"], off, q, k, v, qw, kw, 1, HQ, HKV, D,
                                     False)
            el += time.perf_counter() - t
            n += 1
        ex_q, _, _ = O.producer_f64(dec["pos"], off, q, k, v, qw, kw, 1, HQ, HKV, D, False)
        res["cpu_baseline"] = {"value": round(32 * n / el, 2), "unit": "tokens/s",
                               "cores": 1, "kind": "port", "host": host_cpu_info(),
                               "sample": f"{n} decode-shape calls (32 tokens each) of the "
                                         f"oracle's per-token rms_norm / apply_rope_qk / "
                                         f"append, one thread"}
        res["parity_sample"] = {"q_out_max_rel_err_vs_cpu_fp32":
                                float(f"{O.max_rel_err(got_q, want_q):.3g}"),
                                "q_out_max_rel_err_vs_float64":
                                float(f"{O.max_rel_err(got_q, ex_q):.3g}"),
                                "cpu_fp32_vs_float64": float(f"{O.max_rel_err(want_q, ex_q):.3g}")}
    return res


def bench_lsa(args, log):
    """LSA sparse attention (pkv_attend_sparse) on the model's global-layer geometry (16 q /
    2 kv heads, head_dim 512, fp32 pools) for 32 sequences at contexts U[128, 8192]. Each
    key list comes from lsa_expand_buckets with the engine's defaults
    (…batched.mojo:1261-1264: top_k 256 from 20 picked buckets of up to 32 members, window
    128, 4 sinks), so a query attends about 390 keys scattered over its context."""
    from pkv import LayerSpec, LSABucketCache, PagedKVCache, hip, lsa_expand_buckets, synth

    HQ, HKV, D, BS, B = 16, 2, 512, 16, 32
    TOP_K, PICK, CAP, WINDOW, SINKS = 256, 20, 32, 128, 4
    rng = np.random.default_rng(args.seed)
    ctx = rng.integers(128, 8193, B)
    blocks = (ctx + BS) // BS
    nb = int(blocks.sum())
    stride = int(blocks.max())
    perm = rng.permutation(nb).astype(np.int32)
    tables = np.zeros((B, stride), np.int32)
    lists, off = [], [0]
    lsa = LSABucketCache(B, 8192 + 512)  # one index instance per sequence
    c_sizes = np.zeros((B, lsa.max_buckets), np.int32)
    c_members = np.zeros((B, lsa.max_buckets, CAP), np.int32)
    c_picked = np.zeros((B, PICK), np.int32)
    c_npicked = np.zeros(B, np.int32)
    o = 0
    for s in range(B):
        tables[s, :blocks[s]] = perm[o:o + blocks[s]]
        o += blocks[s]
        pos = int(ctx[s])
        nbk = pos // 16 + 1  # buckets of the closed blocks
        sizes = np.minimum(rng.integers(8, CAP + 1, nbk), pos + 1)
        members = np.zeros((nbk, CAP), np.int64)
        for b in range(nbk):
            members[b, :sizes[b]] = rng.choice(pos + 1, sizes[b], replace=False)
        picked = rng.choice(nbk, min(PICK, nbk), replace=False)
        c_sizes[s, :nbk], c_members[s, :nbk] = sizes, members
        c_picked[s, :picked.size], c_npicked[s] = picked, picked.size
        sel = lsa_expand_buckets(picked, sizes, members, pos, TOP_K, SINKS, WINDOW)
        lists.append(sel)
        off.append(off[-1] + sel.size)
    keys = np.concatenate(lists).astype(np.int32)
    off = np.asarray(off, np.int32)
    n_keys = np.diff(off)
    max_keys = int(n_keys.max())
    stream = hip.Stream()
    cache = PagedKVCache([LayerSpec(HQ, HKV, D)], block_size=BS, num_blocks=nb, max_seqs=B,
                         max_blocks_per_seq=stride, scale=0.0625, stream=stream)
    cache.tables.upload(tables)
    synth.fill_normal(cache.k_pools[0], 301)
    synth.fill_normal(cache.v_pools[0], 302)
    q = synth.normal((B, HQ, D), 303)
    dkeys, doff = hip.DeviceArray.from_numpy(keys), hip.DeviceArray.from_numpy(off)
    out = hip.DeviceArray((B, HQ, D), np.float32)
    ev = _event_pairs(hip, args.steps)

    def step(i, events=None):
        if events:
            events[i][0].record(stream)
        cache.attend_sparse(0, q, dkeys, doff.ptr, max_keys, out)
        if events:
            events[i][1].record(stream)

    for i in range(args.warmup):
        step(i)
    ms = _timed(hip, stream, args.steps, step)
    _timed(hip, stream, args.steps, lambda i: step(i, ev))
    # The timed region holds only back-to-back attention calls (stream + merge launch), so
    # its average per call is the launch duration; an event pair around each call adds a
    # few microseconds of its own at this size (kept as a second figure).
    dur = ms / args.steps
    dur_ev = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    got = out.numpy()
    # The same lists built on the device (pkv_lsa_expand over the bucket cache), alone and
    # chained into the attention.
    lsa.sizes.upload_at(0, c_sizes)
    lsa.members.upload_at(0, c_members)
    dev = [hip.DeviceArray.from_numpy(a) for a in (np.arange(B, dtype=np.int32), c_picked,
                                                   c_npicked, ctx.astype(np.int32))]
    per = LSABucketCache.max_keys(TOP_K, SINKS, WINDOW)
    xk, xo, xs = (hip.DeviceArray((B * per,), np.int32), hip.DeviceArray((B + 1,), np.int32),
                  hip.DeviceArray((B,), np.int32))

    def expand(i, events=None, chain=False):
        if events:
            events[i][0].record(stream)
        lsa.expand(*dev, TOP_K, SINKS, WINDOW, xk, xo, xs, stream=stream)
        if chain:
            cache.attend_sparse(0, q, xk, xo.ptr, per, out)
        if events:
            events[i][1].record(stream)

    for i in range(args.warmup):
        expand(i, chain=True)
    _timed(hip, stream, args.steps, lambda i: expand(i, ev))
    dur_x = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    _timed(hip, stream, args.steps, lambda i: expand(i, ev, chain=True))
    dur_xa = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
    n_off = xo.numpy()
    device_lists_equal = bool(np.array_equal(n_off, off) and
                              np.array_equal(xk.numpy()[:n_off[-1]], keys) and
                              not xs.numpy().any())
    chained = out.numpy()
    chained_diff = float(np.max(np.abs(chained - got) / (np.abs(got) + 1e-3)))
    # each listed key's K and V slices once, Q in / O out, key list and table entries
    nbytes = int(n_keys.sum()) * (2 * HKV * D * 4 + 8) + B * 2 * HQ * D * 4
    res = _line("LSA sparse paged attention tokens/s (32 sequences, ~390-key lists, 16q/2kv/512)",
                B * args.steps / (ms / 1e3), "tokens/s", args.steps, args.warmup,
                ms / args.steps, "f32",
                "LSA decode step on the global-layer geometry: 32 sequences, contexts U[128,8192], "
                "key lists from lsa_expand_buckets (top_k 256 of 20 buckets, window 128, "
                "4 sinks), 16q/2kv/512, block 16, fp32 KV",
                _roofline(nbytes, dur, "stream_attend_kernel<512, float, 2, 4, sparse> + "
                                       "stream_merge_kernel<512, double>"),
                {"launch_us_event_pairs": round(dur_ev * 1e3, 2),
                 "keys_per_sequence_mean": round(float(n_keys.mean()), 1),
                 "max_keys": max_keys,
                 "device_expand": {"us_per_call": round(dur_x * 1e3, 2),
                                   "expand_plus_attend_us": round(dur_xa * 1e3, 2),
                                   "lists_equal_host_expand": device_lists_equal,
                                   "chained_max_rel_diff": float(f"{chained_diff:.3g}")}})
    _set_traffic(res["roofline"], "lsa_sparse_stream_traffic.md")
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        O.use_host_build()

        k = cache.k_pools[0].numpy().reshape(-1)
        v = cache.v_pools[0].numpy().reshape(-1)
        qh = q.numpy()
        n, el, refs = 0, 0.0, []
        while el < args.cpu_seconds and n < B:
            t = time.perf_counter()
            refs.append(O.attend_sparse(qh[n:n + 1], k, v, tables[n:n + 1], keys[off[n]:off[n + 1]],
                                        np.array([0, n_keys[n]], np.int32), HQ, HKV, D, BS,
                                        scale=0.0625, nthreads=args.cpu_threads))
            el += time.perf_counter() - t
            n += 1
        exact = O.attend_sparse_f64(qh[:n], k, v, tables[:n], keys[:off[n]], off[:n + 1], HQ,
                                    HKV, D, BS, scale=0.0625)
        ref = np.concatenate(refs)
        res["cpu_baseline"] = {"value": round(n / el, 2), "unit": "tokens/s",
                               "cores": args.cpu_threads, "kind": "port", "host": host_cpu_info(),
                               "sample": f"first {n} sequences, one lsa_sparse_paged_attention "
                                         f"call each on {args.cpu_threads} head-pair threads"}
        res["parity_sample"] = {"sequences": n,
                                "max_rel_err_vs_cpu_fp32": float(f"{O.max_rel_err(got[:n], ref):.3g}"),
                                "max_rel_err_vs_float64": float(f"{O.max_rel_err(got[:n], exact):.3g}"),
                                "cpu_fp32_vs_float64": float(f"{O.max_rel_err(ref, exact):.3g}")}
    return res


def bench_wo(args, log):
    """The Wo projection after attention (pkv_q4_matmul: Q4_0 weights x attn_out) at the
    decode batch of config 2 (32 sequences), for the sliding layers' 4096 -> 2816 and the
    global layers' 8192 -> 2816 (16 q heads x 256 / 512 -> hidden 2816, config.json)."""
    from pkv import hip, q4_matmul, synth

    B, C_OUT = 32, 2816
    stream = hip.Stream()
    rng = np.random.default_rng(args.seed)
    legs = {}
    for name, c_in in (("sliding", 4096), ("global", 8192)):
        # Q4_0 blocks: seeded random nibbles and positive block scales
        packed = rng.integers(0, 256, (C_OUT, c_in // 2), dtype=np.uint8)
        scales = (rng.random((C_OUT, c_in // 32)) * 0.01 + 0.001).astype(np.float32)
        dw, ds = hip.DeviceArray.from_numpy(packed), hip.DeviceArray.from_numpy(scales)
        x = synth.normal((B, c_in), 401)
        out = hip.DeviceArray((B, C_OUT), np.float32)
        ws = q4_matmul(dw, ds, x, out, c_in, C_OUT, B, stream=stream)
        ev = _event_pairs(hip, args.steps)

        def step(i, events=None):
            if events:
                events[i][0].record(stream)
            q4_matmul(dw, ds, x, out, c_in, C_OUT, B, workspace=ws, stream=stream)
            if events:
                events[i][1].record(stream)

        for i in range(args.warmup):
            step(i)
        ms = _timed(hip, stream, args.steps, step)
        _timed(hip, stream, args.steps, lambda i: step(i, ev))
        # The timed region holds nothing but back-to-back calls of the one kernel, so its
        # average per call is the launch duration; an event pair around each launch adds
        # a few microseconds of its own at this size (kept as a second figure).
        dur = ms / args.steps
        dur_ev = float(np.mean([a.elapsed_ms(b) for a, b in ev]))
        nbytes = C_OUT * c_in // 2 + C_OUT * c_in // 32 * 4 + B * c_in * 4 + B * C_OUT * 4
        legs[name] = dict(ms=ms, dur=dur, dur_ev=dur_ev, nbytes=nbytes, packed=packed,
                          scales=scales, x=x.numpy(), got=out.numpy(), c_in=c_in)
    g, sl = legs["global"], legs["sliding"]
    res = _line("Wo projection (Q4_0) sequences/s at the decode batch, global layer 8192 -> 2816",
                B * args.steps / (g["ms"] / 1e3), "sequences/s", args.steps, args.warmup,
                g["ms"] / args.steps, "q4_0 x f32",
                "pkv_q4_matmul: 32 sequences' attn_out (16 q heads x 512 = 8192) times the Q4_0 "
                "Wo matrix (2816 x 8192, block 32), fp32 out",
                _roofline(g["nbytes"], g["dur"], "q4_matmul_kernel<2, 1, 3>"),
                {"data": "synthetic: seeded N(0,1) x, Q4_0 weights with seeded random nibbles "
                         "and block scales U[0.001, 0.011) (random-init, no checkpoint)",
                 "launch_us_event_pairs": round(g["dur_ev"] * 1e3, 2),
                 "sliding_4096": {"us_per_call": round(sl["dur"] * 1e3, 2),
                                  "gbs": round(sl["nbytes"] / (sl["dur"] / 1e3) / 1e9, 1),
                                  "bytes_per_call": int(sl["nbytes"])}})
    _set_traffic(res["roofline"], "wo_q4_matmul_traffic.md")
    if args.cpu_seconds > 0:
        from oracle import oracle as O

        O.use_host_build()
        n, el = 0, 0.0
        errs = []
        while el < args.cpu_seconds and n < B:
            t = time.perf_counter()
            ref = O.q4_matmul_vec(g["packed"], g["scales"], g["x"][n])
            el += time.perf_counter() - t
            exact = O.q4_matmul_f64(g["packed"], g["scales"], g["x"][n])
            errs.append((float(np.max(np.abs(g["got"][n] - ref))),
                         float(np.max(np.abs(g["got"][n] - exact))),
                         float(np.max(np.abs(ref - exact)))))
            n += 1
        res["cpu_baseline"] = {"value": round(n / el, 2), "unit": "sequences/s", "cores": 1,
                               "kind": "port", "host": host_cpu_info(),
                               "sample": f"{n} q4_matmul_vec calls (8192 -> 2816), one thread"}
        res["parity_sample"] = {"max_abs_err_vs_cpu_fp32": float(f"{max(e[0] for e in errs):.3g}"),
                                "max_abs_err_vs_float64": float(f"{max(e[1] for e in errs):.3g}"),
                                "cpu_fp32_vs_float64": float(f"{max(e[2] for e in errs):.3g}")}
    return res


def kernel_name(sched):
    """The attention kernels a decode schedule's launches run (stream kernel + merge)."""
    if sched.D == 512:  # 8 rows per kv head on the fp64 matrix cores
        return "stream_mfma_kernel<512, 1, 1, 2, paged> (fp64 MFMA) + stream_merge_kernel<512, double>"
    return "stream_attend_kernel<256, float, 2> + stream_merge_kernel<256, double>"


def bench_decode(args, log, sched, metric, workload, traffic_profile):
    """A DecodeSchedule (config 2, or its schedule on another geometry) through
    pkv_append_attend per layer and step; returns the JSON line's dict."""
    from pkv import hip

    t = time.perf_counter()
    data = sched.device_data()
    hip.synchronize()
    L = sched.L
    log(f"decode schedule built in {time.perf_counter() - t:.1f}s: {sched.num_blocks} blocks, "
        f"contexts {sched.ctx0.min()}..{sched.ctx0.max()}")
    g = run_gpu(sched, data, args.steps, args.warmup, log)
    steps = args.steps
    ms_per_step = g["gpu_ms"] / steps
    tok_s = sched.B * steps / (g["gpu_ms"] / 1e3)
    dur, nb = g["dur_ms"], g["bytes"]
    achieved = nb.sum() / (dur.sum() / 1e3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": None,
                "kernel": kernel_name(sched),
                "avg_launch_us": round(dur.mean() * 1e3, 2),
                "algorithmic_bytes_per_launch": int(nb.mean())}
    _set_traffic(roofline, traffic_profile)
    result = {
        "metric": metric, "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded N(0,1) K/V/Q, seeded contexts U[128,8192], seeded "
                "random non-overlapping block tables",
        "config": {"workload": workload, "batch": sched.B, "num_blocks": sched.num_blocks, "head_dim": sched.D,
                   "kv_heads": sched.HKV, "q_heads": sched.HQ, "block_size": sched.BS},
        "roofline": roofline,
        "ms_per_step_with_launch_events": round(g["gpu_ms_ev"] / steps, 4),
        "step_calls": "per layer pkv_append_attend (the attention launch also writes the "
                      "appended rows); roofline pass: pkv_append, then the event pair around "
                      "pkv_attend",
        "wall_s": round(g["wall_s"], 4),
        "append_status_ok": bool(np.all(g["status"] == 0)),
    }
    for layer, win in enumerate(sched.windows):  # per layer: its own bytes over its own launches
        name = "global" if win <= 0 else "sliding"
        gbs = nb[:, layer].sum() / (dur[:, layer].sum() / 1e3) / 1e9
        result[f"attn_{name}_gbs"] = round(gbs, 1)
        result[f"attn_{name}_frac"] = round(gbs / PEAK_HBM_GBS, 4)
        result[f"attn_{name}_avg_us"] = round(dur[:, layer].mean() * 1e3, 2)
    if args.cpu_seconds > 0:
        from oracle import oracle as O

        lib_path = O.use_host_build()
        host = host_cpu_info()
        all_threads = host["omp_num_threads"] or os.cpu_count() or 1
        all_threads = min(all_threads, os.cpu_count() or all_threads)
        c = run_cpu(sched, data, args.cpu_seconds / 2, args.cpu_threads, log, par=0)
        cb = run_cpu(sched, data, args.cpu_seconds / 2, all_threads, log, par=3)
        errs = [O.max_rel_err(g["outs"][j, layer], c["outs"][j][layer])
                for j in range(min(c["steps"], steps)) for layer in range(L)]
        same = all(np.array_equal(c["outs"][j][layer], cb["outs"][j][layer])
                   for j in range(min(c["steps"], cb["steps"])) for layer in range(L))
        faithful = round(sched.B * c["steps"] / c["seconds"], 2)
        batched = round(sched.B * cb["steps"] / cb["seconds"], 2)
        result["cpu_baseline"] = {
            "value": batched, "unit": "tokens/s", "cores": all_threads, "kind": "port",
            "sample": f"first {cb['steps']} steps of the same 64-step schedule (every layer, "
                      f"appends + attention), all-cores batched: every (sequence, head pair) "
                      f"task of a step on {all_threads} threads; the oracle's "
                      f"{os.path.basename(lib_path)} build",
            "host": host,
            "modes": {
                "reference_faithful": {
                    "value": faithful, "threads": args.cpu_threads, "steps": c["steps"],
                    "how": f"sequences in turn, {args.cpu_threads} head-pair tasks per call "
                           f"(attention.mojo:276-287)"},
                "all_cores_batched": {"value": batched, "threads": all_threads,
                                      "steps": cb["steps"],
                                      "outputs_equal_reference_faithful": bool(same)}}}
        if errs:
            result["parity_sample_max_rel_err"] = float(f"{max(errs):.3g}")
            # The fp32 reference path is itself an approximation: on these long contexts it
            # sits ~1e-4 from the exact (float64) attention. The GPU accumulates in double
            # and is held to 1e-5 of float64 (tests/parity.py).
            e64 = [O.max_rel_err(g["outs"][j, layer], ex) for j, layer, ex in c["exact"]]
            own = [O.max_rel_err(c["outs"][j][layer], ex) for j, layer, ex in c["exact"]]
            result["parity_sample"] = {
                "steps": min(c["steps"], steps), "max_rel_err_vs_cpu_fp32": float(f"{max(errs):.3g}"),
                "max_rel_err_vs_float64": float(f"{max(e64):.3g}"),
                "cpu_fp32_vs_float64": float(f"{max(own):.3g}"),
                "float64_steps": len(c["exact"]) // L,
                "metric": "max |x-ref|/(|ref|+1e-3)"}
    return result


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bound on the CPU-baseline sample (0 disables it)")
    ap.add_argument("--cpu-threads", type=int, default=8,
                    help="threads of the reference-faithful CPU mode (8 = its Hq/2 head-pair "
                         "tasks); the all-cores mode uses the job's OpenMP share of the host")
    ap.add_argument("--quiet", action="store_true")
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5],
                    help="BASELINE.json configuration (2, the default, is the headline)")
    ap.add_argument("--kv-dtype", choices=["f32", "bf16"], default="f32",
                    help="pool element type of --config 5 (bf16: the bf16-pool variant)")
    ap.add_argument("--leg", choices=["producer", "lsa", "wo", "global512"], default=None,
                    help="measure a path beside the configurations instead: 'producer' = "
                         "pkv_append_qkv (norm + RoPE + append), 'lsa' = pkv_attend_sparse, "
                         "'wo' = pkv_q4_matmul, 'global512' = config 2's decode schedule on "
                         "the engine's global-layer geometry (16q/2kv/512)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures the paged KV path on one GPU only: every GPU box here has "
              "one GPU and this path has no multi-GPU leg (splitting sequences or heads "
              "across GPUs is not built). Run with --gpus 1.", file=sys.stderr)
        return 2

    def log(msg):
        if not args.quiet:
            print(f"[bench] {msg}", file=sys.stderr, flush=True)

    from pkv import hip
    from pkv.workloads import DecodeSchedule

    if hip.device_count() < 1:
        print("bench.py needs a GPU: no HIP device visible", file=sys.stderr)
        return 1
    if args.leg in ("producer", "lsa", "wo"):
        leg = {"producer": bench_producer, "lsa": bench_lsa, "wo": bench_wo}[args.leg]
        print(json.dumps(leg(args, log)), flush=True)
        return 0
    legs = {1: bench_config1, 3: bench_config3, 4: bench_config4, 5: bench_config5}
    if args.config in legs:
        print(json.dumps(legs[args.config](args, log)), flush=True)
        return 0
    if args.leg == "global512":
        sched = DecodeSchedule.engine_global(seed=args.seed)
        result = bench_decode(
            args, log, sched,
            metric="engine global-layer paged decode tokens/s (16q/2kv/512, B=32, 1 GPU)",
            workload="config 2's schedule on the engine's global-layer geometry: 32 sequences, "
                     "contexts U[128,8192], one full-attention layer, 16q/2kv/512 "
                     "(model_speculative_moe_batched.mojo:1905-1907), block 16, fp32 KV, "
                     "scale 2^-4, retire 4 / admit 4 (256 tok) every 8 steps, "
                     "64-step schedule",
            traffic_profile="stream_decode_global512_traffic.md")
    else:
        sched = DecodeSchedule(seed=args.seed)
        result = bench_decode(
            args, log, sched, metric=METRIC,
            workload="BASELINE config 2: continuous-batching decode, 32 sequences, "
                     "sliding(1024)+global layers, 16q/8kv/256, block 16, fp32 KV, "
                     "retire 4 / admit 4 (256 tok) every 8 steps, 64-step schedule",
            traffic_profile="stream_attend_decode_cfg2_traffic.md")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
