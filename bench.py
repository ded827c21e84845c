#!/usr/bin/env python3
"""Benchmark of the GDN hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline workload: one decode step of the
single-token gated delta rule across 24 GDN layers, batch 64 sequences,
32 value heads / 16 key heads, d_k = d_v = 128, fp32 state.  A step is 24
launches of the decode kernel (one per layer, each with its own 128 MiB
state and inputs), all resident in HBM before timing starts.
value = 64 tokens / step time.

The JSON line also carries:
  roofline      the decode kernel: algorithmic bytes per launch / its mean
                launch time from HIP events on the launch stream, vs 8 TB/s
  cpu_baseline  the CPU oracle (oracle/, OpenMP over (sequence, head)) on a
                bounded sample of the same step, on this host's cores,
                pinned; then on one pinned thread.  The conv, decay and scan
                lines carry their own cpu_baseline: the reference's scalar C
                (compiled from its sources into oracle/_ref) on one pinned
                thread, and the OpenMP port on all cores
  secondary     prefill (config 3, T=16K), the fp16-state prefill at
                T in {1K, 8K, 32K, 128K} (config 4: tokens/s and the per-layer
                state footprint), conv+SiLU (config 1) and cumulative decay
                ([4096][8192]) throughput and roofline, the gated scan and
                the fp16/bf16 scan and decay variants, the layer glue, and
                the hybrid decode loop (config 5: B=1 and B=16, 256 greedy
                steps after a 32K context)
Synthetic inputs with the BASELINE distributions; random state.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s

# Decode
B_DEC, HV, HK, DK, DV, LAYERS = 64, 32, 16, 128, 128, 24
DEC_BYTES = (2 * B_DEC * HV * DK * DV * 4            # state read + write
             + 2 * B_DEC * HK * DK * 4               # q, k
             + 2 * B_DEC * HV * DV * 4               # v, o
             + 2 * B_DEC * HV * 4)                   # g, beta
assert DEC_BYTES == 271_597_568
# Prefill: dense-GEMM FLOPs per (chunk, value head)
PF_T = 16384
PF_WARMUP_S = 0.15  # warm-up time before a prefill line's timed calls (see Timer.p50_ms)
PF_FLOP_PER_CHUNK_HEAD = 5 * (2 * 64 * 64 * 128) + 3 * (2 * 64 * 128 * 128)
assert PF_FLOP_PER_CHUNK_HEAD == 11_534_336
# Conv and decay
CONV_T, CONV_C = 4096, 8192
CONV_BYTES = (2 * CONV_T * CONV_C + 4 * CONV_C + 2 * 3 * CONV_C) * 4
assert CONV_BYTES == 268_763_136
DEC_T, DEC_C = 4096, 8192
DECAY_BYTES = 2 * DEC_T * DEC_C * 4


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def profile_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, scaled by a copy-kernel calibration), when committed."""
    p = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(p) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


class Timer:
    """HIP-event timing on torch's current stream (the stream every entry
    point is called with)."""

    def __init__(self, torch):
        self.torch = torch

    def time_ms(self, fn, reps):
        t = self.torch
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        t.cuda.synchronize()
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        e.synchronize()
        return s.elapsed_time(e) / reps

    def p50_ms(self, fn, warmup=20, reps=30, warmup_s=0.0):
        """The reference's protocol (bench_kai_gdn.c:55-60,86-95): `warmup`
        untimed calls, then `reps` calls timed one by one with HIP events,
        median by nearest rank.  With warmup_s, the untimed calls also go on
        until that much time has passed: after the host-side set-up of a line
        (seconds with the GPU idle) the GPU runs at lowered clocks, and the
        MFMA-bound prefill needs about 100 calls (30 ms) to return to its
        steady rate -- with the reference's 20 warm-ups alone the T=16K line
        read 12% slow (274 against 244 us on one box)."""
        t = self.torch
        for _ in range(warmup):
            fn()
        if warmup_s > 0:
            t0 = time.perf_counter()
            while True:
                for _ in range(10):
                    fn()
                t.cuda.synchronize()
                if time.perf_counter() - t0 >= warmup_s:
                    break
        ev = [t.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        t.cuda.synchronize()
        for i in range(reps):
            ev[i].record()
            fn()
        ev[reps].record()
        ev[reps].synchronize()
        ts = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(reps))
        return ts[(reps - 1) // 2]

    def per_call_ms(self, fns):
        """Each callable of `fns` run once, in order, with an event recorded
        between consecutive calls on the launch stream; returns the list of
        per-call durations (each kernel's own launch time)."""
        t = self.torch
        ev = [t.cuda.Event(enable_timing=True) for _ in range(len(fns) + 1)]
        t.cuda.synchronize()
        ev[0].record()
        for i, fn in enumerate(fns):
            fn()
            ev[i + 1].record()
        ev[-1].synchronize()
        return [ev[i].elapsed_time(ev[i + 1]) for i in range(len(fns))]



def bench_decode(L, ob, torch, steps, warmup, timer, f16_state=False, warmup_s=0.0):
    """The configs[1] step: 24 launches of the decode kernel, one per layer,
    each with its own state (fp32, or fp16 with f16_state: the narrow-state
    variant of row a6, half the state bytes).  `warmup` untimed steps, then,
    with warmup_s, untimed steps until that much time has passed: the
    inputs' host-side set-up leaves the GPU idle for seconds, and a 0.6 ms
    step needs more than five steps to return to its steady clock (the first
    20 timed fp16-state steps after 10 warm-ups read 25.2 us per launch
    against a steady 24.2)."""
    from tests.gdn_inputs import decode_inputs
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    qs = 1.0 / math.sqrt(DK)
    layers = []
    for l in range(LAYERS):
        S, q, k, v, g, beta = decode_inputs(1000 + l, B_DEC, HV, HK, DK, DV)
        t = {n: torch.from_numpy(a).cuda() for n, a in
             dict(S=S, q=q, k=k, v=v, g=g, beta=beta).items()}
        if f16_state:
            t["S"] = t["S"].half().view(torch.int16)
        t["o"] = torch.empty((B_DEC, HV, DV), dtype=torch.float32, device="cuda")
        layers.append(t)
    torch.cuda.synchronize()
    fn = L.kai_run_gdn_delta_rule_decode_f16state_hip if f16_state else L.kai_run_gdn_delta_rule_decode_f32_hip

    def launch(t):
        rc = fn(t["S"].data_ptr(), t["q"].data_ptr(), t["k"].data_ptr(), t["v"].data_ptr(),
                t["g"].data_ptr(), t["beta"].data_ptr(), t["o"].data_ptr(), B_DEC, HV, HK, DK,
                DV, qs, stream)
        if rc:
            ob.check(rc, "decode")

    def step():
        for t in layers:
            launch(t)

    for _ in range(warmup):
        step()
    t0 = time.perf_counter()
    while warmup_s > 0 and time.perf_counter() - t0 < warmup_s:
        step()
        torch.cuda.synchronize()
    ms_step = timer.time_ms(step, steps)
    # The timed region holds only decode launches, back to back on the
    # stream the events are recorded on: its time / launch count is the mean
    # launch duration (the rocprofv3 average agrees within 1%).  Events
    # recorded between every pair of launches, the alternative, add each
    # event's own cost (about 3 us) to every launch; that figure is kept as
    # a cross-check.
    kern_ms = ms_step / LAYERS
    durs = timer.per_call_ms([(lambda t=t: launch(t)) for _ in range(min(steps, 20)) for t in layers])
    return ms_step, kern_ms, sum(durs) / len(durs)


def cpu_sets():
    """The CPUs the CPU legs are pinned to: the first omp_get_max_threads()
    CPUs this process may run on (all cores), and the first of them alone
    (one thread)."""
    from oracle import oracle as orc
    allowed = sorted(os.sched_getaffinity(0))
    return allowed[:max(1, min(orc.num_threads(), len(allowed)))], allowed


def pin(cpus):
    """What `taskset -a -p` does: pin every thread of this process (OpenMP
    workers included; threads started later inherit the mask) to `cpus`."""
    for tid in os.listdir("/proc/self/task"):
        try:
            os.sched_setaffinity(int(tid), set(cpus))
        except OSError:
            pass


def cpu_p50_ms(fn, budget_s, min_reps=3, max_reps=30):
    """One untimed call, then calls timed one by one until `budget_s` is
    spent (at least `min_reps`, at most `max_reps`); median by nearest rank,
    the GPU protocol's statistic.  Returns (p50 ms, calls timed, seconds)."""
    fn()
    ts, t_start = [], time.perf_counter()
    while len(ts) < max_reps and (len(ts) < min_reps or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    ts.sort()
    return ts[(len(ts) - 1) // 2], len(ts), time.perf_counter() - t_start


def cpu_stream_baseline(budget_s=1.0):
    """CPU legs of the [4096][8192] stream lines (conv, decay, scans):
    - "reference": the reference's own portable C, compiled from its sources
      by oracle/Makefile into oracle/_ref (kai ukernels' scalar branches for
      the fp32 conv, decay and scan; gdn_sve.c for the fp16/bf16 scan and
      decay), one thread pinned to one core;
    - "port": this repo's C restatement (oracle/, OpenMP over channels) on
      all cores, pinned.
    The kai conv has no SiLU, so the conv line's reference leg is the conv
    alone; the port runs conv+SiLU, the GPU line's workload.  Inputs have
    the GPU lines' distributions: the conv inputs of config 1; decay factors
    exp(-softplus(N(0,1)) exp(U(-2,0))) for the fp32 decay; gates U(0,1)
    and x N(0,1) for the scans and the narrow decays."""
    from oracle import oracle as orc
    from tests.gdn_inputs import conv_inputs
    P = orc.P
    T, C = DEC_T, DEC_C
    cx, w, hist = (np.ascontiguousarray(v, dtype=np.float32) for v in conv_inputs(1, CONV_T, CONV_C))
    rs = np.random.RandomState(2)
    gl = -np.log1p(np.exp(rs.randn(T * C))) * np.exp(rs.uniform(-2, 0, T * C))
    a = np.exp(gl).astype(np.float32)
    del gl
    x = rs.randn(T * C).astype(np.float32)
    g = rs.uniform(0.0, 1.0, T * C).astype(np.float32)
    out = np.empty(T * C, np.float32)
    out16 = np.empty(T * C, np.uint16)
    st32 = np.zeros(C, np.float32)
    st16 = np.zeros(C, np.uint16)
    z = (ctypes.c_size_t(T), ctypes.c_size_t(C))
    kai, sve, port = orc.ref_kai(), orc.ref_sve(), orc.lib()
    scan32 = 3 * T * C * 4 + 2 * C * 4
    scan16 = 3 * T * C * 4 + 2 * C * 2
    # line name: (bytes, reference (lib, symbol, args) or None, port (symbol, args))
    jobs = {
        "conv": (CONV_BYTES, (kai, "kai_run_gdn_causal_dwconv1d_f32_k4_sve", (P(cx), P(w), P(out), P(hist))),
                 ("orc_causal_dwconv1d_silu_f32_k4", (P(cx), P(w), P(out), P(hist)))),
        "cumdecay": (DECAY_BYTES, (kai, "kai_run_gdn_cumdecay_f32_sve", (P(a), P(out))),
                     ("orc_cumdecay_f32", (P(a), P(out)))),
        "gated_scan_f32": (scan32, (kai, "kai_run_gdn_gated_scan_f32_sve", (P(g), P(x), P(out), P(st32))),
                           ("orc_gated_scan_f32", (P(g), P(x), P(out), P(st32)))),
        "gated_scan_f16": (scan16, (sve, "gdn_gated_scan_f16", (P(g), P(x), P(out), P(st16))),
                           ("orc_gated_scan_f16", (P(g), P(x), P(out), P(st16)))),
        "gated_scan_bf16": (scan16, (sve, "gdn_gated_scan_bf16", (P(g), P(x), P(out), P(st16))),
                            ("orc_gated_scan_bf16", (P(g), P(x), P(out), P(st16)))),
        "cumdecay_f16": (T * C * 6, (sve, "gdn_cumdecay_f16", (P(g), P(out16))),
                         ("orc_cumdecay_f16", (P(g), P(out16)))),
        "cumdecay_bf16": (T * C * 6, (sve, "gdn_cumdecay_bf16", (P(g), P(out16))),
                          ("orc_cumdecay_bf16", (P(g), P(out16)))),
    }
    all_cpus, allowed = cpu_sets()
    threads = orc.num_threads()
    res = {}
    for name, (nbytes, ref, (psym, pargs)) in jobs.items():
        entry = {"unit": "GB/s", "cpu_model": cpu_model()}
        pin(all_cpus)
        pfn = getattr(port, psym)
        ms, n, el = cpu_p50_ms(lambda: pfn(*pargs, *z), budget_s)
        port_leg = {"value": round(nbytes / (ms * 1e-3) / 1e9, 2), "us": round(ms * 1e3, 1),
                    "cores": len(all_cpus), "kind": "port",
                    "sample": f"{psym}, [{T}][{C}], p50 of {n} calls ({el:.1f} s), "
                              f"{threads} OpenMP threads pinned to CPUs {all_cpus[0]}-{all_cpus[-1]}"}
        lib, rsym, rargs = ref
        if lib is not None:
            pin(all_cpus[:1])
            orc.set_num_threads(1)
            rfn = getattr(lib, rsym)
            ms, n, el = cpu_p50_ms(lambda: rfn(*rargs, *z), budget_s)
            orc.set_num_threads(threads)
            entry.update({"value": round(nbytes / (ms * 1e-3) / 1e9, 3), "us": round(ms * 1e3, 1),
                          "cores": 1, "kind": "reference",
                          "sample": f"{rsym} (reference source, oracle/_ref build, -O3), [{T}][{C}], "
                                    f"p50 of {n} calls ({el:.1f} s), one thread pinned to CPU {all_cpus[0]}"})
            entry["port_all_cores"] = port_leg
        else:
            entry.update(port_leg)
            entry["note"] = "oracle/_ref not built: the port is the baseline"
        res[name] = entry
    pin(allowed)
    return res


def cpu_decode_baseline(budget_s=12.0, single_budget_s=10.0):
    """The oracle (OpenMP over (sequence, head)) on the same per-layer step,
    pinned to the cores it uses; runs whole layers until the budget is spent,
    reports tokens/s of a 24-layer step.  Then the same on one thread
    (OpenMP set to 1, pinned to one core)."""
    from oracle import oracle as orc
    from tests.gdn_inputs import decode_inputs
    S, q, k, v, g, beta = decode_inputs(1000, B_DEC, HV, HK, DK, DV)

    def run(budget, cap):
        nonlocal S
        orc.delta_rule_decode(S, q, k, v, g, beta, B_DEC, HV, HK, DK, DV, 1 / math.sqrt(DK))
        n, t0 = 0, time.perf_counter()
        while True:
            S, _ = orc.delta_rule_decode(S, q, k, v, g, beta, B_DEC, HV, HK, DK, DV, 1 / math.sqrt(DK))
            n += 1
            el = time.perf_counter() - t0
            if el > budget or n >= cap:
                return n, el

    threads = orc.num_threads()
    all_cpus, allowed = cpu_sets()
    pin(all_cpus)
    n, el = run(budget_s, 2400)
    pin(all_cpus[:1])
    orc.set_num_threads(1)
    n1, el1 = run(single_budget_s, 240)
    orc.set_num_threads(threads)
    pin(allowed)
    return {"value": round(B_DEC / (el / n * LAYERS), 2), "unit": "tokens/s",
            "cores": len(all_cpus), "kind": "port",
            "sample": f"{n} layer-steps of B=64 x 32 heads x 128x128 fp32 "
                      f"({n / LAYERS:.1f} full 24-layer steps), {el:.1f} s, {threads} OpenMP threads "
                      f"pinned to CPUs {all_cpus[0]}-{all_cpus[-1]}",
            "single_thread": {"value": round(B_DEC / (el1 / n1 * LAYERS), 2), "cores": 1,
                              "sample": f"{n1} layer-steps, {el1:.1f} s, pinned to CPU {all_cpus[0]}"},
            "cpu_model": cpu_model()}


def bench_prefill(L, ob, torch, timer, reps=5):
    from tests.gdn_inputs import bf16_bits, prefill_inputs
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    q, k, v, g, beta, S = prefill_inputs(7, 1, PF_T, HV, HK)
    dq, dk_, dv_ = (torch.from_numpy(bf16_bits(x).view(np.int16)).cuda() for x in (q, k, v))
    dg, db, dS = (torch.from_numpy(x).cuda() for x in (g, beta, S))
    do = torch.empty((1, PF_T, HV, 128), dtype=torch.int16, device="cuda")
    fn = L.kai_run_gdn_chunk_delta_rule_bf16_f32_hip

    def run():
        rc = fn(dq.data_ptr(), dk_.data_ptr(), dv_.data_ptr(), dg.data_ptr(), db.data_ptr(),
                do.data_ptr(), dS.data_ptr(), 1, PF_T, HV, HK, 1 / math.sqrt(128), stream)
        if rc:
            ob.check(rc, "prefill")

    ms_ref = timer.p50_ms(run, warmup=20, reps=max(reps, 30))
    ms = timer.p50_ms(run, warmup=20, reps=max(reps, 30), warmup_s=PF_WARMUP_S)
    windowed = int(L.kai_gdn_hip_prefill_windowed_heads())
    # the same shapes with long-memory gates: g = -0.01 (the state decays by
    # e^-0.64 per chunk, 2^-24 in 26 chunks: windows that long), and
    # g = -0.001 (no window within a segment bounds it: the exact two-pass
    # path)
    dg.fill_(-0.01)
    ms_long = timer.p50_ms(run, warmup=20, reps=max(reps, 30), warmup_s=PF_WARMUP_S)
    long_windowed = int(L.kai_gdn_hip_prefill_windowed_heads())
    dg.fill_(-0.001)
    ms_exact = timer.p50_ms(run, warmup=20, reps=max(reps, 30), warmup_s=PF_WARMUP_S)
    exact_windowed = int(L.kai_gdn_hip_prefill_windowed_heads())
    flop = PF_FLOP_PER_CHUNK_HEAD * (PF_T // 64) * HV
    tflops = flop / (ms * 1e-3) / 1e12
    return {"workload": "chunked WY prefill, B=1 T=16384 Hv=32 Hk=16 d=128 bf16 in, fp32 state",
            "tokens_per_s": round(PF_T / (ms * 1e-3), 1), "ms": round(ms, 4),
            "achieved_tflops": round(tflops, 2), "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            "flop_per_launch": flop, "ms_20_warmups": round(ms_ref, 4),
            "windowed_heads": windowed,
            "ms_long_memory": round(ms_long, 4), "long_memory_windowed_heads": long_windowed,
            "ms_exact_path": round(ms_exact, 4), "exact_path_windowed_heads": exact_windowed,
            "mfma_frac_exact_path": round(flop / (ms_exact * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
            "timing_note": f"ms: p50 of 30 calls after {PF_WARMUP_S:g} s of warm-up calls (steady clocks); "
                           "ms_20_warmups: the reference's 20 warm-ups alone, right after the input "
                           "set-up left the GPU idle (clocks still rising)"}


def device_prefill_inputs(torch, seed, T, Hv, Hk, d=128):
    """Synthetic prefill inputs with the BASELINE distributions, generated on
    the GPU (the long-sequence lines would take minutes on the host): q, k
    L2-normalised N(0,1) and v ~ N(0,1), as bf16 bit patterns in int16
    tensors; g = -softplus(N(0,1)) exp(U(-2,0)), beta = sigmoid(N(0,1)),
    S ~ N(0, 0.02), fp32."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    F = torch.nn.functional

    def nrm(*shape):
        return torch.randn(*shape, generator=gen, device="cuda")

    q = F.normalize(nrm(1, T, Hk, d), dim=-1).to(torch.bfloat16).view(torch.int16)
    k = F.normalize(nrm(1, T, Hk, d), dim=-1).to(torch.bfloat16).view(torch.int16)
    v = nrm(1, T, Hv, d).to(torch.bfloat16).view(torch.int16)
    beta = torch.sigmoid(nrm(1, T, Hv))
    g = -F.softplus(nrm(1, T, Hv)) * torch.exp(
        torch.rand(1, T, Hv, generator=gen, device="cuda") * 2.0 - 2.0)
    S = 0.02 * nrm(1, Hv, d, d)
    return q, k, v, g.contiguous(), beta.contiguous(), S


def bench_prefill_f16_state(L, ob, torch, timer, lengths=(1024, 8192, 32768, 131072)):
    """Config 4: the chunked prefill with an fp16 recurrent state (fp32
    accumulation) at growing T; the state a layer keeps between calls is
    Hv x 128 x 128 fp16 whatever T is."""
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    fn = L.kai_run_gdn_chunk_delta_rule_bf16_f16state_hip
    rows = []
    for T in lengths:
        q, k, v, g, beta, S = device_prefill_inputs(torch, 40 + T // 1024, T, HV, HK)
        S16 = S.half().view(torch.int16)
        o = torch.empty((1, T, HV, 128), dtype=torch.int16, device="cuda")

        def run():
            rc = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                    o.data_ptr(), S16.data_ptr(), 1, T, HV, HK, 1 / math.sqrt(128), stream)
            if rc:
                ob.check(rc, "prefill fp16 state")

        ms = timer.p50_ms(run, warmup=20, reps=30, warmup_s=PF_WARMUP_S)
        flop = PF_FLOP_PER_CHUNK_HEAD * ((T + 63) // 64) * HV
        state_b = S16.numel() * S16.element_size()
        carry_b = int(L.kai_gdn_hip_prefill_workspace_bytes(1, T, HV))
        rows.append({"T": T, "ms": round(ms, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
                     "achieved_tflops": round(flop / (ms * 1e-3) / 1e12, 2),
                     "state_bytes_per_layer": state_b, "carry_bytes": carry_b,
                     "footprint_bytes_one_layer": state_b + carry_b,
                     "library_device_bytes_held": int(L.kai_gdn_hip_device_bytes_held())})
        del q, k, v, g, beta, S, S16, o
    return {"workload": "chunked WY prefill with fp16 state (fp32 accumulate), B=1 Hv=32 Hk=16 "
                        "d=128, bf16 q/k/v (BASELINE configs[3])",
            "footprint_note": "state_bytes_per_layer: the fp16 state tensor a layer keeps between calls "
                              "(measured from the allocation); carry_bytes: the library's segment carry "
                              "buffer for this T (one per device, shared by all layers, whose calls run "
                              "one after another); library_device_bytes_held: all device memory the "
                              "library holds after the call (the carry buffer grown with 25% headroom, "
                              "scan status arrays, staging)",
            "state_bytes_per_layer_fp32_state": HV * 128 * 128 * 4,
            "lengths": rows}


def bench_layer_glue(L, ob, torch, timer, T=PF_T):
    """The layer glue at the prefill shape (B=1, T=16384, Hk=16, Hv=32):
    the gating prologue (conv output fp32 -> q, k, v bf16, g, beta) and the
    bf16 gated RMSNorm over the T * Hv rows of the recurrence output.  Both
    are HBM-bound; bytes are each kernel's reads plus writes."""
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(31)
    H = 2 * HK + HV
    x = torch.randn(T, H * 128, generator=gen, device="cuda")
    a = torch.randn(T, HV, generator=gen, device="cuda")
    b = torch.randn(T, HV, generator=gen, device="cuda")
    A_log = torch.log(torch.rand(HV, generator=gen, device="cuda") * 15 + 0.5)
    dt = torch.randn(HV, generator=gen, device="cuda")
    q = torch.empty(T, HK, 128, dtype=torch.int16, device="cuda")
    k = torch.empty_like(q)
    v = torch.empty(T, HV, 128, dtype=torch.int16, device="cuda")
    g = torch.empty(T, HV, device="cuda")
    beta = torch.empty_like(g)

    def prologue():
        rc = L.kai_run_gdn_gating_prologue_bf16_hip(
            x.data_ptr(), a.data_ptr(), b.data_ptr(), A_log.data_ptr(), dt.data_ptr(),
            q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), T, HK, HV,
            stream)
        if rc:
            ob.check(rc, "gating prologue")

    ms = timer.p50_ms(prologue, warmup=20, reps=30)
    pro_bytes = T * H * 128 * 4 + 2 * T * HV * 4 + 2 * HV * 4 + T * H * 128 * 2 + 2 * T * HV * 4
    pro = {"workload": f"gating prologue, B=1 T={T} Hk={HK} Hv={HV}: fp32 conv output -> "
                       "L2-normalised q, k and v (bf16), g, beta",
           "us": round(ms * 1e3, 2), "tokens_per_s": round(T / (ms * 1e-3), 1),
           "bytes_per_launch": pro_bytes, "achieved_gbs": round(pro_bytes / (ms * 1e-3) / 1e9, 1),
           "hbm_frac": round(pro_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del x, a, b, q, k, v, g, beta
    rows = T * HV
    o = torch.randn(rows, 128, generator=gen, device="cuda").to(torch.bfloat16)
    z = torch.randn(rows, 128, generator=gen, device="cuda").to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(128, generator=gen, device="cuda")).to(torch.bfloat16)
    y = torch.empty_like(o)

    def norm():
        rc = L.kai_run_gdn_gated_rmsnorm_bf16_hip(o.data_ptr(), z.data_ptr(), w.data_ptr(),
                                                  y.data_ptr(), rows, 1e-6, stream)
        if rc:
            ob.check(rc, "gated rmsnorm")

    ms = timer.p50_ms(norm, warmup=20, reps=30)
    rn_bytes = 3 * rows * 128 * 2 + 128 * 2
    rn = {"workload": f"gated RMSNorm + SiLU(z), bf16, {rows} rows of 128 (B=1 T={T} Hv={HV})",
          "us": round(ms * 1e3, 2), "tokens_per_s": round(T / (ms * 1e-3), 1),
          "bytes_per_launch": rn_bytes, "achieved_gbs": round(rn_bytes / (ms * 1e-3) / 1e9, 1),
          "hbm_frac": round(rn_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return pro, rn


HYB_CONTEXT, HYB_STEPS = 32768, 256


def hybrid_step_bytes(cfg, weight_bytes, B, pos):
    """HBM bytes one decode step of the hybrid model must move at position
    pos: every int8 weight matrix with its scales once, the embedding rows,
    the fp16 K and V caches up to pos + 1 (plus the appended row), and each
    GDN layer's fp32 recurrent state (read + write) and conv state."""
    attn = cfg.layers // cfg.attn_every
    gdn = cfg.layers - attn
    conv_dim = 2 * cfg.gdn_k_heads * 128 + cfg.gdn_v_heads * 128
    kv = attn * B * cfg.attn_kv_heads * (pos + 1) * 256 * 2 * 2
    state = gdn * B * (cfg.gdn_v_heads * 128 * 128 * 4 * 2 + conv_dim * 4 * 4 * 2)
    return weight_bytes + B * cfg.hidden * 2 + kv + state


def hybrid_prefill_flop(cfg, B, T):
    """Dense FLOPs of a T-token prefill of B sequences: every matmul but the
    LM head (2 x params x tokens; the LM head runs on the last position
    only), the causal attention (q k^T and p v over T (T + 1) / 2 pairs per
    query head) and the chunked delta rule (the prefill metric's per-chunk
    count)."""
    attn = cfg.layers // cfg.attn_every
    gdn = cfg.layers - attn
    H, I = cfg.hidden, cfg.inter
    conv_dim = 2 * cfg.gdn_k_heads * 128 + cfg.gdn_v_heads * 128
    vdim = cfg.gdn_v_heads * 128
    gdn_params = H * (conv_dim + vdim + 2 * cfg.gdn_v_heads) + vdim * H
    attn_params = H * (cfg.attn_q_heads * 512 + 2 * cfg.attn_kv_heads * 256) + cfg.attn_q_heads * 256 * H
    mlp = 3 * H * I
    params = gdn * gdn_params + attn * attn_params + cfg.layers * mlp
    gemm = 2 * params * B * T + 2 * H * cfg.vocab * B
    att = attn * B * cfg.attn_q_heads * 2 * 2 * 256 * (T * (T + 1) // 2)
    delta = gdn * B * cfg.gdn_v_heads * ((T + 63) // 64) * PF_FLOP_PER_CHUNK_HEAD
    return gemm + att + delta


def bench_hybrid(torch, timer, batches=(1, 16), context=HYB_CONTEXT, steps=HYB_STEPS, kind="prefilled"):
    """the Qwen3.5-4B-shaped hybrid model (24 GDN + 8
    attention layers, int8 per-output-channel weights, fp16 activations and
    KV cache), greedy decoding of `steps` tokens per sequence after a
    `context`-token context, batch 1 and 16; tokens never leave the device
    (each step's argmax feeds the next), the decode loop timed with HIP
    events around it.  The context:
      prefilled  a prefill of `context` uniform-random token ids per
                 sequence (kai_gdn_hybrid_prefill), timed on its own: the
                 time to first token (the prefill's last position yields the
                 first generated token);
      drawn      drawn states (KV caches, recurrent and conv states);
      stepped    the random ids stepped through the decode loop (untimed)."""
    from orionsbelt_amd import hybrid as hb
    rows = []
    for B in batches:
        cfg = hb.qwen35_4b(B, context + steps + 1)
        m = hb.HybridModel(cfg, 12345)
        m.reset(B, context, 7)
        tok = torch.randint(0, cfg.vocab, (B,), dtype=torch.int32, device="cuda")
        nxt = torch.empty_like(tok)
        logits = torch.empty(B, cfg.vocab, dtype=torch.float32, device="cuda")
        for _ in range(3):  # warm-up steps, then a fresh context
            m.step(tok, nxt, logits)
        extra = {}
        if kind == "prefilled":
            gen = torch.Generator(device="cuda")
            gen.manual_seed(2026)
            prompt = torch.randint(0, cfg.vocab, (B, context), dtype=torch.int32, device="cuda", generator=gen)
            m.prefill(prompt[:, :256].contiguous(), nxt, logits)  # warm-up: buffers, code
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            m.prefill(prompt, tok, logits)  # the first generated token lands in tok
            e.record()
            e.synchronize()
            pms = s.elapsed_time(e)
            flop = hybrid_prefill_flop(cfg, B, context)
            extra = {"ttft_ms": round(pms, 2), "prefill_tokens_per_s": round(B * context / (pms * 1e-3), 1),
                     "prefill_flop": int(flop), "prefill_achieved_tflops": round(flop / (pms * 1e-3) / 1e12, 1)}
            extra["prefill_mfma_frac"] = round(extra["prefill_achieved_tflops"] / BF16_PEAK_TFLOPS, 4)
            log(f"  B={B}: prefill of {context} tokens per sequence in {pms:.1f} ms")
            del prompt
        elif kind == "stepped":
            m.reset(B, 0, 7)
            gen = torch.Generator(device="cuda")
            gen.manual_seed(2026)
            prompt = torch.randint(0, cfg.vocab, (context, B), dtype=torch.int32, device="cuda", generator=gen)
            t0 = time.perf_counter()
            for t in range(context):
                m.step(prompt[t], None, None)
                if (t + 1) % 4096 == 0:
                    torch.cuda.synchronize()
                    log(f"  B={B}: {t + 1} context tokens stepped")
            torch.cuda.synchronize()
            log(f"  B={B}: stepped a {context}-token context in {time.perf_counter() - t0:.1f} s")
            tok.copy_(prompt[-1])
            del prompt
        else:
            m.reset(B, context, 7)
        assert m.position == context
        bufs = [tok, nxt]

        def run():
            for i in range(steps):
                m.step(bufs[i & 1], bufs[(i + 1) & 1], logits)

        ms = timer.time_ms(run, 1)
        per = ms / steps
        nbytes = sum(hybrid_step_bytes(cfg, m.weight_bytes, B, context + i) for i in range(steps)) / steps
        gbs = nbytes / (per * 1e-3) / 1e9
        rows.append({"batch": B, "context": context, "context_kind": kind, **extra,
                     "steps": steps, "ms_per_step": round(per, 4),
                     "tokens_per_s": round(B / (per * 1e-3), 1), "bytes_per_step": int(nbytes),
                     "achieved_gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                     "device_bytes": m.device_bytes})
        m.close()
        del m, logits, tok, nxt, bufs
        torch.cuda.empty_cache()
    what = {"prefilled": "a prefilled", "stepped": "a stepped", "drawn": "a drawn"}[kind]
    return {"workload": f"hybrid decode loop, Qwen3.5-4B shape (32 layers: 24 GDN + 8 attention, hidden 2560, "
                        f"inter 9216, vocab 151936), int8 weights, fp16 activations and KV cache, greedy, "
                        f"{steps} steps after {what} {context}-token context of uniform-random ids "
                        f"(BASELINE configs[4]); ttft_ms: the prefill's time, the first token included",
            "runs": rows}


def cpu_prefill_baseline(budget_s=10.0):
    from oracle import oracle as orc
    from tests.gdn_inputs import prefill_inputs
    T = 256
    q, k, v, g, beta, S = prefill_inputs(7, 1, T, HV, HK)
    all_cpus, allowed = cpu_sets()
    pin(all_cpus)
    n, t0 = 0, time.perf_counter()
    while True:
        orc.chunk_gdr(q, k, v, g, beta, S, 1, T, HV, HK, 128, 128, 64)
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s:
            break
    pin(allowed)
    return {"value": round(n * T / el, 1), "unit": "tokens/s", "cores": len(all_cpus),
            "kind": "port", "sample": f"{n} x T={T} (32 heads, OpenMP over heads), {el:.1f} s, "
                                      f"pinned to CPUs {all_cpus[0]}-{all_cpus[-1]}",
            "cpu_model": cpu_model()}


def bench_stream(L, ob, torch, timer, reps=40, sets=4):
    """conv+SiLU and cumdecay at [4096][8192], rotating `sets` distinct
    buffer sets (1 GiB) so no launch is served by the 256 MB Infinity Cache."""
    from tests.gdn_inputs import conv_inputs
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x, w, h = conv_inputs(1, CONV_T, CONV_C)
    dx = [torch.from_numpy(x).cuda() for _ in range(sets)]
    dw, dh = torch.from_numpy(w).cuda(), torch.from_numpy(h).cuda()
    do = [torch.empty(CONV_T * CONV_C, dtype=torch.float32, device="cuda") for _ in range(sets)]
    it = [0]

    def conv():
        j = it[0] % sets
        it[0] += 1
        rc = L.kai_run_gdn_causal_dwconv1d_silu_f32_k4_hip(dx[j].data_ptr(), dw.data_ptr(),
                                                          do[j].data_ptr(), dh.data_ptr(), CONV_T,
                                                          CONV_C, stream)
        if rc:
            ob.check(rc, "conv")

    for _ in range(sets):
        conv()
    conv_ms = timer.time_ms(conv, reps)
    del dx, do
    rs = np.random.RandomState(2)
    gl = -np.log1p(np.exp(rs.randn(DEC_T * DEC_C))) * np.exp(rs.uniform(-2, 0, DEC_T * DEC_C))
    a = np.exp(gl).astype(np.float32)
    da = [torch.from_numpy(a).cuda() for _ in range(sets)]
    dd = [torch.empty(DEC_T * DEC_C, dtype=torch.float32, device="cuda") for _ in range(sets)]

    def decay():
        j = it[0] % sets
        it[0] += 1
        rc = L.kai_run_gdn_cumdecay_f32_hip(da[j].data_ptr(), dd[j].data_ptr(), DEC_T, DEC_C,
                                            stream)
        if rc:
            ob.check(rc, "cumdecay")

    for _ in range(sets):
        decay()
    dec_ms = timer.time_ms(decay, reps)
    if L.kai_gdn_hip_check_device_error() != 0:
        raise RuntimeError("cumdecay look-back watchdog fired")
    conv_gbs = CONV_BYTES / (conv_ms * 1e-3) / 1e9
    dec_gbs = DECAY_BYTES / (dec_ms * 1e-3) / 1e9
    return (
        {"workload": "causal dwconv1d K=4 + SiLU, T=4096 C=8192 fp32", "us": round(conv_ms * 1e3, 2),
         "tokens_per_s": round(CONV_T / (conv_ms * 1e-3), 1), "achieved_gbs": round(conv_gbs, 1),
         "hbm_frac": round(conv_gbs / HBM_PEAK_GBS, 4)},
        {"workload": "cumulative decay [4096][8192] fp32", "us": round(dec_ms * 1e3, 2),
         "achieved_gbs": round(dec_gbs, 1), "hbm_frac": round(dec_gbs / HBM_PEAK_GBS, 4)},
    )


def bench_scans(L, ob, torch, timer, reps=40, sets=4):
    """The diagonal gated scan (row a3) and the narrow-state variants of the
    scan and of the cumulative decay (row a6) at [4096][8192], rotating
    `sets` buffer sets (over 1.5 GiB).  Bytes per launch: the scan reads g
    and x and writes s ([T][C] fp32 each) and reads and writes its state
    ([C], fp32 or 2-byte); the narrow decay reads a (fp32) and writes decay
    (2-byte)."""
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    T, C = DEC_T, DEC_C
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    gs = [torch.rand(T * C, generator=gen, device="cuda") for _ in range(sets)]
    xs = [torch.randn(T * C, generator=gen, device="cuda") for _ in range(sets)]
    ss = [torch.empty(T * C, device="cuda") for _ in range(sets)]
    st32 = torch.zeros(C, device="cuda")
    st16 = torch.zeros(C, dtype=torch.int16, device="cuda")
    d16 = [torch.empty(T * C, dtype=torch.int16, device="cuda") for _ in range(sets)]
    it = [0]
    out = {}

    def run(name, fn, nbytes, narrow):
        def call():
            j = it[0] % sets
            it[0] += 1
            rc = fn(j)
            if rc:
                ob.check(rc, name)

        for _ in range(sets):
            call()
        ms = timer.time_ms(call, reps)
        if L.kai_gdn_hip_check_device_error() != 0:
            raise RuntimeError(f"{name}: look-back watchdog fired")
        gbs = nbytes / (ms * 1e-3) / 1e9
        what = "output" if name.startswith("cumdecay") else "state"
        out[name] = {"workload": f"{name.replace('_', ' ')} [{T}][{C}]" + (f", {narrow} {what}" if narrow else ""),
                     "us": round(ms * 1e3, 2), "bytes_per_launch": nbytes, "achieved_gbs": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}

    scan32 = 3 * T * C * 4 + 2 * C * 4
    scan16 = 3 * T * C * 4 + 2 * C * 2
    run("gated_scan_f32", lambda j: L.kai_run_gdn_gated_scan_f32_hip(
        gs[j].data_ptr(), xs[j].data_ptr(), ss[j].data_ptr(), st32.data_ptr(), T, C, stream), scan32, None)
    run("gated_scan_f16", lambda j: L.kai_run_gdn_gated_scan_f16_hip(
        gs[j].data_ptr(), xs[j].data_ptr(), ss[j].data_ptr(), st16.data_ptr(), T, C, stream), scan16, "fp16")
    run("gated_scan_bf16", lambda j: L.kai_run_gdn_gated_scan_bf16_hip(
        gs[j].data_ptr(), xs[j].data_ptr(), ss[j].data_ptr(), st16.data_ptr(), T, C, stream), scan16, "bf16")
    run("cumdecay_f16", lambda j: L.kai_run_gdn_cumdecay_f16_hip(
        gs[j].data_ptr(), d16[j].data_ptr(), T, C, stream), T * C * 6, "fp16")
    run("cumdecay_bf16", lambda j: L.kai_run_gdn_cumdecay_bf16_hip(
        gs[j].data_ptr(), d16[j].data_ptr(), T, C, stream), T * C * 6, "bf16")
    del gs, xs, ss, d16
    torch.cuda.empty_cache()
    return out


def measure_peaks(L, ob, torch, timer):
    """What this GPU delivers, measured with the library's probes
    (kai_gdn_hip_probe_*): a 2 GiB streaming copy (bytes read + written), a
    4 GiB streaming read, and independent bf16 MFMA chains (32x32x16, and
    16x16x32) on 16 blocks per CU.  Both buffers exceed the 256 MB Infinity
    Cache."""
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sink = torch.empty(L.kai_gdn_hip_probe_sink_bytes() // 4 + 1, dtype=torch.float32, device="cuda")
    nb = 2 << 30
    src = torch.empty(nb // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1.0)

    def copy():
        ob.check(L.kai_gdn_hip_probe_stream(src.data_ptr(), dst.data_ptr(), nb, 0, sink.data_ptr(), stream), "probe")

    ms = timer.p50_ms(copy, warmup=3, reps=10)
    copy_gbs = 2 * nb / (ms * 1e-3) / 1e9
    del dst
    big = torch.empty((4 << 30) // 4, dtype=torch.float32, device="cuda")
    big.fill_(1.0)

    def read():
        ob.check(L.kai_gdn_hip_probe_stream(big.data_ptr(), None, big.numel() * 4, 1, sink.data_ptr(), stream),
                 "probe")

    ms = timer.p50_ms(read, warmup=3, reps=10)
    read_gbs = big.numel() * 4 / (ms * 1e-3) / 1e9
    del big, src
    flops = ctypes.c_ulonglong(0)
    tflops = []
    for shape in (0, 1):
        def mfma():
            ob.check(L.kai_gdn_hip_probe_mfma_bf16(2000, shape, sink.data_ptr(), ctypes.byref(flops), stream),
                     "probe")

        ms = timer.p50_ms(mfma, warmup=3, reps=10)
        tflops.append(flops.value / (ms * 1e-3) / 1e12)
    torch.cuda.empty_cache()
    return {"hbm_copy_gbs": round(copy_gbs, 1), "hbm_read_gbs": round(read_gbs, 1),
            "mfma_bf16_tflops": round(tflops[0], 1), "mfma_bf16_16x16x32_tflops": round(tflops[1], 1),
            "note": "measured on this GPU with kai_gdn_hip_probe_*: 2 GiB copy (bytes read + written), 4 GiB "
                    "read, bf16 MFMA 32x32x16 chains (and 16x16x32, the prefill's instruction); the "
                    "roofline fractions use the datasheet peaks, the *_measured fractions these"}


def add_measured_fracs(d, peaks, read_bound=False):
    """frac_measured next to every hbm_frac / mfma_frac of a result tree."""
    if isinstance(d, list):
        for x in d:
            add_measured_fracs(x, peaks, read_bound)
        return
    if not isinstance(d, dict):
        return
    if "achieved_gbs" in d:
        ref = peaks["hbm_read_gbs"] if read_bound else peaks["hbm_copy_gbs"]
        d["hbm_frac_measured"] = round(d["achieved_gbs"] / ref, 4)
    if "achieved_tflops" in d:
        d["mfma_frac_measured"] = round(d["achieved_tflops"] / peaks["mfma_bf16_tflops"], 4)
    for v in d.values():
        if isinstance(v, (dict, list)):
            add_measured_fracs(v, peaks, read_bound)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def run_profile(which, L, ob, torch, timer, steps, warmup):
    """Workload for rocprofv3: `which`, then a plain copy kernel
    (dst = src * 1 over 64M fp32: reads and writes exactly 268,435,456 bytes),
    the reference for scaling FETCH_SIZE / WRITE_SIZE to bytes."""
    if which == "decode":
        ms, kern, pairs = bench_decode(L, ob, torch, steps, warmup, timer)
        log(f"decode: {ms:.4f} ms/step, {kern * 1e3:.2f} us/launch ({pairs * 1e3:.2f} with events between launches)")
    elif which == "prefill":
        log(f"prefill: {bench_prefill(L, ob, torch, timer, reps=steps)}")
    elif which == "prefill_f16":
        log(f"prefill fp16 state: {bench_prefill_f16_state(L, ob, torch, timer)}")
    elif which == "layer":
        pro, rn = bench_layer_glue(L, ob, torch, timer)
        log(f"gating prologue: {pro}\ngated rmsnorm: {rn}")
    elif which == "hybrid":
        log(f"hybrid (prefilled context): {bench_hybrid(torch, timer, steps=steps)}")
    elif which == "hybrid_drawn":
        log(f"hybrid (drawn context): {bench_hybrid(torch, timer, steps=steps, kind='drawn')}")
    elif which == "hybrid_real":
        log(f"hybrid (stepped context): {bench_hybrid(torch, timer, steps=steps, kind='stepped')}")
    else:
        conv, decay = bench_stream(L, ob, torch, timer, reps=steps)
        log(f"{which}: {conv if which == 'conv' else decay}")
    src = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    log("calibration copy: 3 x 268435456 bytes")


def compact_cpu(c):
    """A cpu_baseline entry without its long strings (they stay on the
    detail line)."""
    if not c:
        return c
    out = {k: c[k] for k in ("value", "unit", "cores", "kind") if k in c}
    if "sample" in c:  # its first clause, without parentheses
        out["sample"] = re.sub(r"\s*\([^)]*\)", "", c["sample"]).split(",")[0]
    if "single_thread" in c:
        out["single_thread"] = c["single_thread"]["value"]
    if "port_all_cores" in c:
        out["port_all_cores"] = c["port_all_cores"]["value"]
    return out


def compact_secondary(sec):
    """The secondary lines, figures only, in a fixed order with the T=16K
    prefill (the second half of the metric) last."""
    out = {}

    def stream_line(d):
        e = {"us": d.get("us"), "frac": d.get("hbm_frac")}
        c = d.get("cpu_baseline")
        if c:  # GB/s of the reference's scalar build (1 core) and of the port (all cores)
            if c.get("kind") == "reference":
                e["cpu_ref_gbs"] = c["value"]
                e["cpu_port_gbs"] = c["port_all_cores"]["value"]
            else:
                e["cpu_port_gbs"] = c["value"]
        return e

    for key in ("conv", "cumdecay"):
        if key in sec:
            out[key] = stream_line(sec[key])
    for key, d in sec.get("scans", {}).items():
        out[key] = stream_line(d)
    if "decode_f16_state" in sec:
        d = sec["decode_f16_state"]
        out["decode_f16_state"] = {"ms_per_step": d["ms_per_step"], "tok_s": d["tokens_per_s"],
                                   "launch_us": d["launch_us"], "frac": d["hbm_frac"]}
    for key in ("gating_prologue", "gated_rmsnorm"):
        if key in sec:
            out[key] = stream_line(sec[key])
    if "prefill_f16_state" in sec:
        out["prefill_f16_state"] = [{"T": r["T"], "ms": r["ms"], "tok_s": r["tokens_per_s"],
                                     "state_bytes": r["state_bytes_per_layer"]}
                                    for r in sec["prefill_f16_state"]["lengths"]]
    if "hybrid_decode" in sec:
        out["hybrid_decode"] = [{k: r[k] for k in ("batch", "ms_per_step", "tokens_per_s", "hbm_frac", "ttft_ms")
                                 if k in r} for r in sec["hybrid_decode"]["runs"]]
    if "prefill" in sec:
        d = sec["prefill"]
        e = {"T": PF_T, "ms": d["ms"], "ms_20_warmups": d["ms_20_warmups"], "tok_s": d["tokens_per_s"],
             "mfma_frac": d["mfma_frac"], "windowed_heads": d["windowed_heads"],
             "ms_long_memory": d.get("ms_long_memory"), "ms_exact_path": d["ms_exact_path"],
             "mfma_frac_exact_path": d["mfma_frac_exact_path"],
             "roofline": {"bound": "mfma",
                          "kernel": "prefill_window_check_kernel+prefill_pass1_kernel+prefill_pass2_kernel",
                          "flop_per_launch": d["flop_per_launch"], "achieved": d["achieved_tflops"],
                          "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": d["mfma_frac"],
                          "traffic": profile_traffic("prefill_windowed_call")}}
        if "cpu_baseline" in d:
            e["cpu_baseline"] = compact_cpu(d["cpu_baseline"])
        out["prefill"] = e
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="skip prefill/conv/decay lines")
    ap.add_argument("--profile", choices=["decode", "prefill", "prefill_f16", "layer", "conv", "cumdecay",
                                          "hybrid", "hybrid_drawn", "hybrid_real"],
                    help="run only this workload (and a 256 MiB device copy that calibrates "
                         "HBM byte counters) for rocprofv3; prints no JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the GDN path has no cross-GPU "
              f"communication; --gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)

    import torch
    import orionsbelt_amd as ob
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    L = ob.lib()
    ob.check(L.kai_gdn_hip_init(), "init")
    timer = Timer(torch)
    if args.profile:
        run_profile(args.profile, L, ob, torch, timer, args.steps, args.warmup)
        return

    log("measured ceilings (copy, read, MFMA probes) ...")
    peaks = measure_peaks(L, ob, torch, timer)
    log(f"peaks: {peaks}")
    log("decode: 24 layers x B=64 ...")
    ms_step, kern_ms, kern_pairs = bench_decode(L, ob, torch, args.steps, args.warmup, timer)
    achieved = DEC_BYTES / (kern_ms * 1e-3) / 1e9
    log(f"decode: {ms_step:.3f} ms/step, kernel {kern_ms * 1e3:.1f} us ({achieved:.0f} GB/s)")

    secondary = {}
    if not args.no_secondary:
        log("prefill T=16K ...")
        secondary["prefill"] = bench_prefill(L, ob, torch, timer)
        log(f"prefill: {secondary['prefill']}")
        log("prefill, fp16 state, T = 1K .. 128K ...")
        secondary["prefill_f16_state"] = bench_prefill_f16_state(L, ob, torch, timer)
        log(f"prefill fp16 state: {secondary['prefill_f16_state']}")
        log("conv / decay ...")
        secondary["conv"], secondary["cumdecay"] = bench_stream(L, ob, torch, timer)
        log(f"conv: {secondary['conv']}\ncumdecay: {secondary['cumdecay']}")
        log("decode with fp16 state ...")
        ms16, kern16, pairs16 = bench_decode(L, ob, torch, args.steps, args.warmup, timer, f16_state=True,
                                             warmup_s=0.15)
        b16 = DEC_BYTES - B_DEC * HV * DK * DV * 4  # the state read + written at 2 bytes
        gbs16 = b16 / (kern16 * 1e-3) / 1e9
        secondary["decode_f16_state"] = {
            "workload": "decode step, 24 layers, B=64, Hv=32 Hk=16, 128x128 fp16 state (fp32 arithmetic)",
            "ms_per_step": round(ms16, 4), "tokens_per_s": round(B_DEC / (ms16 * 1e-3), 1),
            "bytes_per_launch": b16, "launch_us": round(kern16 * 1e3, 2),
            "launch_us_event_pairs": round(pairs16 * 1e3, 2), "achieved_gbs": round(gbs16, 1),
            "hbm_frac": round(gbs16 / HBM_PEAK_GBS, 4)}
        log(f"decode fp16 state: {secondary['decode_f16_state']}")
        log("gated scan and narrow-state scan/decay ...")
        secondary["scans"] = bench_scans(L, ob, torch, timer)
        log(f"scans: {secondary['scans']}")
        log("layer glue (gating prologue, gated RMSNorm) ...")
        secondary["gating_prologue"], secondary["gated_rmsnorm"] = bench_layer_glue(L, ob, torch, timer)
        log(f"gating prologue: {secondary['gating_prologue']}\n"
            f"gated rmsnorm: {secondary['gated_rmsnorm']}")
        log("hybrid model: 32K-token prefill, then the decode loop, B=1 and B=16 ...")
        secondary["hybrid_decode"] = bench_hybrid(torch, timer)
        log(f"hybrid decode: {secondary['hybrid_decode']}")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle) ...")
        cpu = cpu_decode_baseline()
        log(f"cpu: {cpu}")
        if not args.no_secondary:
            secondary["prefill"]["cpu_baseline"] = cpu_prefill_baseline()
            log("cpu baselines of the stream lines (reference scalar build, port) ...")
            stream_cpu = cpu_stream_baseline()
            for name, entry in stream_cpu.items():
                line_ = secondary["scans"].get(name) or secondary.get(name)
                line_["cpu_baseline"] = entry
            log(f"cpu stream: {stream_cpu}")

    rl = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
          "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profile_traffic("delta_decode_kernel"),
          "kernel": "delta_decode_kernel<128,128,f32>", "bytes_per_launch": DEC_BYTES,
          "launch_us": round(kern_ms * 1e3, 2), "launch_us_event_pairs": round(kern_pairs * 1e3, 2),
          "frac_measured": round(achieved / peaks["hbm_copy_gbs"], 4)}
    # launch_us: the timed region (decode launches only, back to back) / launch
    # count; launch_us_event_pairs: events recorded between every two launches,
    # which adds each event's own cost.
    for key, val in secondary.items():
        add_measured_fracs(val, peaks, read_bound=(key == "hybrid_decode"))
    # The whole result tree (workload strings, samples, notes) on stderr; the
    # JSON line on stdout keeps the figures only, with the T=16K prefill last.
    log("detail: " + json.dumps({"roofline": rl, "cpu_baseline": cpu, "measured_peaks": peaks,
                                 "secondary": secondary}))
    line = {
        "metric": "GDN decode tok/s (B=64, 24 layers, 1 GPU) + % of HBM roofline",
        "value": round(B_DEC / (ms_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (BASELINE distributions, random state)",
        "config": {"workload": "gated delta-rule decode step: 24 GDN layers, batch 64, "
                               "Hv=32 Hk=16 d_k=d_v=128, fp32 state (BASELINE configs[1])"},
        "roofline": rl,
        "cpu_baseline": compact_cpu(cpu),
        "peaks": {"copy_gbs": peaks["hbm_copy_gbs"], "read_gbs": peaks["hbm_read_gbs"],
                  "mfma_tflops": peaks["mfma_bf16_tflops"],
                  "mfma16_tflops": peaks["mfma_bf16_16x16x32_tflops"]},
        "secondary": compact_secondary(secondary),
    }
    print(json.dumps(line, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
