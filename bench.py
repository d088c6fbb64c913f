#!/usr/bin/env python3
"""Benchmark of the Gated DeltaNet path on one MI355X.

Headline (the JSON line's ``value``): chunked gated-delta-rule prefill
throughput in tokens/s on the 32k-token varlen workload (16 sequences,
lengths uniform in [512, 4096] -> 35,846 tokens, Hk 16 / Hv 32, d 128,
chunk 64, bf16 q/k/v, fp32 g/beta and state).  The same line carries the
recurrent decode step (batch 256, fp32 state gathered from a 1024-slot
cache, HBM GB/s), the varlen causal conv1d (8 sequences, 19,762 tokens,
8192 channels, width 4), the conv decode update (batch 256) and the fused
decode step (conv update + L2 norm + gating + recurrent step, batch 256,
with the same step as separate ops timed beside it), and the neighbouring
full-attention layers' causal varlen prefill (the same 16 sequence lengths,
Hq 16 / Hkv 2, d 256) and paged decode (batch 256, contexts U[512, 4096],
16-token pages), each with its roofline and, where it applies, the CPU
oracle timed on this host.  Beside the datasheet peaks, the default run
measures two ceilings of this device (a bf16 8192^3 GEMM through hipBLASLt and
a 1 GiB copy by a plain HIP streaming kernel) and gives each roofline as a
fraction of the matching one too.

A step is one call of the op on inputs already resident in HBM.  Timing:
the workload's step runs untimed for ``--settle-ms`` of wall time (default
300 ms; on an idle GPU the first ~50 launches of a sustained load run in the
power controller's start-up transient, e.g. the prefill at ~515 us against
~430 us settled), then W untimed warm-up steps, then K steps bracketed by
device synchronisation;
per-launch kernel time from HIP events recorded on the stream the kernel is
launched on, reported as the median over the K launches (``kernel_ms``, the
figure the rooflines use) with the mean beside it (``kernel_ms_mean``).  The
CPU baselines run torch on os.cpu_count() threads, or on the CPUs the process
is confined to where that is fewer (affinity mask, cgroup quota); each
reports all of these and lscpu's model name.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_MFMA_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
HK, HV, DK, DV, CHUNK = 16, 32, 128, 128, 64
# algorithmic FLOPs per prefill token: KK^T and QK^T once per k-head (C x C x K),
# per v-head w, u, A_qk v', w S, k^T v', q S (2 C V + C K + 3 K V), x2 for FMA
PREFILL_FLOP_PER_TOKEN = 2 * (2 * CHUNK * DK * HK + (2 * CHUNK * DV + CHUNK * DK + 3 * DK * DV) * HV)
# HBM bytes per launch of each kernel on this benchmark's workloads, from
# rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE (KiB per dispatch), each
# scaled by what the same counter reads on a plain 1 GiB streaming copy
# (--workload hbm_copy: FETCH_SIZE x 2.0, WRITE_SIZE x 1.0 on MI355X; the
# factor 2 is exact for 128-byte read requests, which FETCH_SIZE counts as 64
# bytes here, and the request-size counters show these kernels issue almost
# nothing else).  Values from the committed profiles of the current kernels
# (profiles/*.md, which give the commands); a kernel without an entry reports None.
HBM_TRAFFIC_PER_LAUNCH = {
    "gdn_chunk_prefill_kernel": 1_027_048_208,
    "gdn_chunk_prefill_kernel/short": 3_853_347_984,
    "gdn_recurrent_step_kernel": 1_083_263_120,
    "causal_conv1d_varlen_kernel": 666_022_912,
    "causal_conv1d_step_kernel": 59_316_992,
    "gdn_decode_fused_kernel": 1_131_415_744,
    "attn_prefill_kernel": 932_966_560,
    "attn_decode_kernel": 1_257_835_584,  # with its combine kernel
    "attn_paged_prefill_kernel": 822_067_328,
}


def _traffic(kernel: str):
    return HBM_TRAFFIC_PER_LAUNCH.get(kernel)


def _cpu_model() -> str:
    """The host CPU's full identification: /proc/cpuinfo's model name, lscpu's
    model and BIOS model names where they differ from it, and the family /
    model / stepping numbers (lscpu alone prints only "AMD EPYC" on some hosts)."""
    import subprocess

    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    if fields:
                        break
                    continue
                k, v = (x.strip() for x in line.split(":", 1))
                if k in ("model name", "cpu family", "model", "stepping") and k not in fields:
                    fields[k] = v
    except OSError:
        pass
    lscpu = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                lscpu.setdefault(k, v)
    except (OSError, subprocess.SubprocessError):
        pass
    name = fields.get("model name") or lscpu.get("Model name") or "unknown"
    extra = [f"{label} {lscpu[k]}" for k, label in (("Model name", "lscpu"), ("BIOS Model name", "BIOS"))
             if lscpu.get(k) and lscpu[k] != name]
    if "cpu family" in fields:
        extra.append(f"family {fields['cpu family']} model {fields.get('model', '?')} "
                     f"stepping {fields.get('stepping', '?')}")
    return name + (f" ({'; '.join(extra)})" if extra else "")


def _cpu_info() -> dict:
    """The host's CPUs as the CPU baseline sees them: os.cpu_count(), the CPUs
    this process may run on (affinity mask), the cgroup CPU quota, and the
    thread count used: os.cpu_count() unless the process is confined to fewer
    CPUs, where more threads than CPUs would time contention, not the CPU."""
    info = {"os_cpu_count": os.cpu_count() or 1, "model": _cpu_model()}
    usable = info["os_cpu_count"]
    try:
        info["affinity_cpus"] = len(os.sched_getaffinity(0))
        usable = min(usable, info["affinity_cpus"])
    except (AttributeError, OSError):
        info["affinity_cpus"] = None
    info["cgroup_cpu_quota"] = None
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            info["cgroup_cpu_quota"] = int(quota) / int(period)
            usable = min(usable, max(1, int(info["cgroup_cpu_quota"])))
    except (OSError, ValueError):
        pass
    info["threads"] = usable
    return info


_CPU_INFO = None


def _cpu_setup() -> dict:
    """Set torch's CPU thread count for a CPU baseline; returns the CPU info."""
    global _CPU_INFO
    if _CPU_INFO is None:
        _CPU_INFO = _cpu_info()
    torch.set_num_threads(_CPU_INFO["threads"])
    _CPU_INFO["torch_threads"] = torch.get_num_threads()
    return _CPU_INFO


def _cpu_baseline(value, unit, sample) -> dict:
    info = _cpu_setup()
    return {"value": value, "unit": unit, "cores": info["torch_threads"], "kind": "port", "sample": sample,
            "os_cpu_count": info["os_cpu_count"], "affinity_cpus": info["affinity_cpus"],
            "cgroup_cpu_quota": info["cgroup_cpu_quota"], "torch_threads": info["torch_threads"],
            "cpu_model": info["model"]}


class Timing:
    """ms per step over the timed region, and the per-launch kernel time from
    the per-step events: median (the reported figure) and mean."""

    def __init__(self, step_ms: float, per: list, back_to_back_ms: float | None = None):
        self.step_ms = step_ms
        srt = sorted(per)
        n = len(srt)
        self.median_ms = srt[n // 2] if n % 2 else 0.5 * (srt[n // 2 - 1] + srt[n // 2])
        self.mean_ms = sum(per) / n
        self.back_to_back_ms = back_to_back_ms

    def fields(self) -> dict:
        return {"ms_per_step": self.step_ms, "kernel_ms": self.median_ms, "kernel_ms_mean": self.mean_ms}


SETTLE_MS = 300.0  # untimed run of each workload before its warm-up (--settle-ms)
_SLEEP_CYCLES_PER_MS = None


def _sleep_cycles_per_ms() -> float:
    """Rate of torch.cuda._sleep's cycle counter, measured once with events."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        stream = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 1_000_000
        torch.cuda._sleep(n)  # warm
        torch.cuda.synchronize()
        a.record(stream)
        torch.cuda._sleep(n)
        b.record(stream)
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = n / max(a.elapsed_time(b), 1e-3)
    return _SLEEP_CYCLES_PER_MS


def _settle(fn, ms: float) -> None:
    """Run fn untimed for `ms` of wall time, so the timed launches see the
    clock the power controller settles on under this load rather than its
    start-up transient."""
    if ms <= 0:
        return
    t_end, i = time.perf_counter() + ms * 1e-3, 0
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def _time_gpu(fn, steps: int, warmup: int, back_to_back: bool = False) -> Timing:
    """Run fn() warmup + steps times; return the Timing of the timed steps
    (per-step HIP events on the launch stream).  The settle run (SETTLE_MS of
    wall time) comes first.  Before the timed steps, untimed launches of the
    same step keep the stream busy while the host enqueues the timed ones, so
    those run back to back (a launch shorter than the host's enqueue time would
    otherwise be timed with the host's gaps) and the GPU stays under the same
    load throughout (an idle stretch, such as a sleep kernel, lets the power
    controller boost the clock again and the timed launches then start in its
    transient).  With back_to_back, a second pass of `steps` launches runs with
    no events between them (one pair around the pass): for a launch of a few
    microseconds the per-step events add several microseconds each, while the
    pass's mean is the launch's time plus only the queue's gap between kernels."""
    _settle(fn, SETTLE_MS)
    stream = torch.cuda.current_stream()
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n_probe = max(warmup, 1)
    w0.record(stream)
    for i in range(n_probe):
        fn(i)
    w1.record(stream)
    torch.cuda.synchronize()
    per_ms = max(w0.elapsed_time(w1) / n_probe, 1e-3)
    # the host enqueues a step (its events included) in well under 60 us; a
    # step shorter than that cannot keep ahead of the host, so its timed steps
    # wait behind a sleep kernel of about the enqueue time instead
    host_ms = 0.06
    short = per_ms < host_ms and hasattr(torch.cuda, "_sleep")
    pre = 2 if short else min(256, int(steps * host_ms / per_ms) + 2)
    sleep_cycles = int((0.2 + steps * host_ms) * _sleep_cycles_per_ms()) if short else 0
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    base = n_probe
    for j in range(pre):
        fn(base + j)
    base += pre
    if short:
        torch.cuda._sleep(sleep_cycles)
    t0.record(stream)
    for i in range(steps):
        evs[i][0].record(stream)
        fn(base + i)
        evs[i][1].record(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    total = t0.elapsed_time(t1)
    base += steps
    b2b = None
    if back_to_back:
        for j in range(pre):
            fn(base + j)
        base += pre
        if short:
            torch.cuda._sleep(sleep_cycles)
        t0.record(stream)
        for i in range(steps):
            fn(base + i)
        t1.record(stream)
        torch.cuda.synchronize()
        b2b = t0.elapsed_time(t1) / steps
    return Timing(total / steps, [a.elapsed_time(b) for a, b in evs], b2b)


def _time_cpu(fn, budget_s: float, max_reps: int = 5):
    fn()  # warm
    reps, t_start = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t_start
        if el >= budget_s or reps >= max_reps:
            return el / reps


def bench_prefill(dev, steps, warmup, cpu_budget):
    from myvllm_amd import chunk_gated_delta_rule
    from myvllm_amd.workloads import prefill_32k_case

    case = prefill_32k_case()
    T = case.tokens
    q, k, v, g, beta, state, idx, cu = (t.to(dev) for t in (case.q, case.k, case.v, case.g, case.beta,
                                                             case.state, case.idx, case.cu))

    def step(_):
        chunk_gated_delta_rule(q, k, v, g, beta, state, idx, cu)

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms
    flop = PREFILL_FLOP_PER_TOKEN * T
    achieved = flop / (kern_ms * 1e-3) / 1e12
    res = {
        "tokens": T,
        "ms_per_step": ms,
        "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms,
        "tokens_per_s": T / (ms * 1e-3),
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / PEAK_MFMA_TFLOPS, "traffic": _traffic("gdn_chunk_prefill_kernel"),
                     "flop_per_launch": flop, "kernel": "gdn_chunk_prefill_kernel"},
    }
    if cpu_budget > 0:
        from oracle.gdn import chunk_gated_delta_rule_ref

        _cpu_setup()
        st = case.state.clone()
        sec = _time_cpu(lambda: chunk_gated_delta_rule_ref(case.q, case.k, case.v, case.g, case.beta, st, case.idx,
                                                           case.cu, dtype=torch.float32), cpu_budget)
        res["cpu_baseline"] = _cpu_baseline(T / sec, "tokens/s",
                                            f"full workload ({T} tokens), fp32 chunked (C=64) torch restatement")
    return res


def prefill_bytes(case) -> int:
    """Algorithmic HBM bytes of one prefill launch: q, k, v and g, beta read,
    o written, and each (sequence, v-head) state read and written once."""
    el = lambda t: t.numel() * t.element_size()
    n_state = case.idx.numel() * case.state.shape[1] * case.state.shape[2] * case.state.shape[3] * 4
    return el(case.q) + el(case.k) + 2 * el(case.v) + el(case.g) + el(case.beta) + 2 * n_state


def bench_prefill_short(dev, steps, warmup, cpu_budget):
    from myvllm_amd import chunk_gated_delta_rule
    from myvllm_amd.workloads import prefill_short_case

    case = prefill_short_case()
    T = case.tokens
    q, k, v, g, beta, state, idx, cu = (t.to(dev) for t in (case.q, case.k, case.v, case.g, case.beta,
                                                             case.state, case.idx, case.cu))

    def step(_):
        chunk_gated_delta_rule(q, k, v, g, beta, state, idx, cu)

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms
    nbytes = prefill_bytes(case)
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    res = {
        "tokens": T, "sequences": int(case.idx.numel()),
        "ms_per_step": ms,
        "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms,
        "tokens_per_s": T / (ms * 1e-3),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": _traffic("gdn_chunk_prefill_kernel/short"),
                     "bytes_per_launch": nbytes, "kernel": "gdn_chunk_prefill_kernel",
                     "mfma_TFLOP_per_s": PREFILL_FLOP_PER_TOKEN * T / (kern_ms * 1e-3) / 1e12},
    }
    if cpu_budget > 0:
        from oracle.gdn import chunk_gated_delta_rule_ref

        _cpu_setup()
        n = 64  # a bounded sample: the first 64 sequences
        cu_s = case.cu[: n + 1]
        Ts = int(cu_s[-1])
        st = case.state.clone()
        sec = _time_cpu(lambda: chunk_gated_delta_rule_ref(case.q[:Ts], case.k[:Ts], case.v[:Ts], case.g[:Ts],
                                                           case.beta[:Ts], st, case.idx[:n], cu_s,
                                                           dtype=torch.float32), cpu_budget)
        res["cpu_baseline"] = _cpu_baseline(Ts / sec, "tokens/s",
                                            f"first {n} of the {case.idx.numel()} sequences ({Ts} tokens), "
                                            "fp32 chunked (C=64) torch restatement")
    return res


def bench_prefill_skewed(dev, steps, warmup, cpu_budget):
    """A chunked-prefill scheduler's batch with one long prompt chunk among
    many short ones: 384 sequences of 64 tokens and one of 16,384 (40,960
    tokens), Hk 16 / Hv 32, d 128.  The launcher takes the many-items
    schedule (two chunks or fewer per sequence on average); its runs are
    priced by tokens, so the long sequence's 32 items spread over workgroups.
    The same batch is also timed with one item per workgroup, longest first
    (gdn_chunk_prefill_ex, items_per_wg = 0), for comparison."""
    from myvllm_amd import chunk_gated_delta_rule
    from myvllm_amd.gated_delta_rule import chunk_prefill_ex
    from myvllm_amd.workloads import prefill_case

    lengths = [64] * 384 + [16384]
    case = prefill_case(lengths, seed=7, num_slots=len(lengths))
    T = case.tokens
    q, k, v, g, beta, state, idx, cu = (t.to(dev) for t in (case.q, case.k, case.v, case.g, case.beta,
                                                             case.state, case.idx, case.cu))
    o = torch.empty(v.shape, dtype=v.dtype, device=dev)

    def step(_):
        chunk_gated_delta_rule(q, k, v, g, beta, state, idx, cu, out=o)

    def step_one_item(_):
        chunk_prefill_ex(q, k, v, g, beta, state, idx, cu, o, DK ** -0.5, items_per_wg=0)

    tm = _time_gpu(step, steps, warmup)
    tm1 = _time_gpu(step_one_item, steps, warmup)
    nbytes = prefill_bytes(case)
    gbs = nbytes / (tm.median_ms * 1e-3) / 1e9
    return {
        "tokens": T, "sequences": len(lengths), **tm.fields(),
        "tokens_per_s": T / (tm.step_ms * 1e-3),
        "one_item_per_workgroup_kernel_ms": tm1.median_ms,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": gbs / PEAK_HBM_GBS, "traffic": None, "bytes_per_launch": nbytes,
                     "kernel": "gdn_chunk_prefill_kernel"},
    }


def bench_decode(dev, steps, warmup, cpu_budget):
    from myvllm_amd import recurrent_gated_delta_rule
    from myvllm_amd.workloads import decode_case

    B, slots = 256, 1024
    case = decode_case(B=B, num_slots=slots, seed=0, state=False)
    gen = torch.Generator(device=dev).manual_seed(0)
    state = torch.randn(slots, HV, DK, DV, device=dev, generator=gen) * 0.1
    # 4 disjoint slot sets in rotation, so the 256 MB last-level cache cannot serve repeats
    perm = torch.randperm(slots, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    idxs = [perm[i * B:(i + 1) * B].to(dev) for i in range(4)]
    q, k, v, g, beta = (t.to(dev) for t in (case.q, case.k, case.v, case.g, case.beta))

    def step(i):
        recurrent_gated_delta_rule(q, k, v, g, beta, state, idxs[i % 4])

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms
    per_seq = 2 * HV * DK * DV * 4 + (2 * HK * DK + 2 * HV * DV) * 2 + 2 * HV * 4 + 4
    nbytes = per_seq * B
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    res = {
        "batch": B,
        "ms_per_step": ms,
        "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms,
        "GB_per_s": gbs,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": _traffic("gdn_recurrent_step_kernel"), "bytes_per_launch": nbytes,
                     "kernel": "gdn_recurrent_step_kernel"},
    }
    if cpu_budget > 0:
        from oracle.gdn import recurrent_gated_delta_rule_ref

        _cpu_setup()
        sub = 32  # bounded sample: 32 of the 256 sequences (64 MB of state)
        st = torch.randn(sub, HV, DK, DV) * 0.1
        sidx = torch.arange(sub, dtype=torch.int32)
        sec = _time_cpu(lambda: recurrent_gated_delta_rule_ref(case.q[:sub], case.k[:sub], case.v[:sub], case.g[:sub],
                                                               case.beta[:sub], st, sidx, dtype=torch.float32),
                        cpu_budget)
        res["cpu_baseline"] = _cpu_baseline(per_seq * sub / sec / 1e9, "GB/s",
                                            f"{sub} of {B} sequences, fp32 token recurrence")
    return res


def bench_conv(dev, steps, warmup, cpu_budget):
    from myvllm_amd import causal_conv1d_fn
    from myvllm_amd.workloads import CONV_DIM, CONV_WIDTH, conv_prefill_case

    case = conv_prefill_case()
    T, D, W, N = int(case.cu[-1]), CONV_DIM, CONV_WIDTH, case.cu.numel() - 1
    x, w, st, idx, cu = (t.to(dev) for t in (case.x, case.weight, case.state, case.idx, case.cu))

    def step(_):
        causal_conv1d_fn(x, w, st, idx, cu)

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms
    nbytes = 4 * T * D + 2 * D * W + 2 * N * (W - 1) * D * 4
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    res = {"tokens": T, "ms_per_step": ms, "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms, "GB_per_s": gbs,
           "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                        "frac": gbs / PEAK_HBM_GBS, "traffic": _traffic("causal_conv1d_varlen_kernel"),
                        "bytes_per_launch": nbytes, "kernel": "causal_conv1d_varlen_kernel"}}
    if cpu_budget > 0:
        from oracle.conv import causal_conv1d_fn_ref

        _cpu_setup()
        cst = case.state.clone()
        sec = _time_cpu(lambda: causal_conv1d_fn_ref(case.x, case.weight, cst, case.idx, case.cu, dtype=torch.float32),
                        cpu_budget)
        res["cpu_baseline"] = _cpu_baseline(nbytes / sec / 1e9, "GB/s", "full workload, fp32 F.conv1d + SiLU per sequence")
    return res


def bench_conv_update(dev, steps, warmup, cpu_budget):
    from myvllm_amd import causal_conv1d_update
    from myvllm_amd.workloads import CONV_DIM, CONV_WIDTH, conv_decode_case

    case = conv_decode_case()
    B, D, W = case.x.shape[0], CONV_DIM, CONV_WIDTH
    x, w, st = (t.to(dev) for t in (case.x, case.weight, case.state))
    perm = torch.randperm(1024, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    idxs = [perm[i * B:(i + 1) * B].to(dev) for i in range(4)]

    def step(i):
        causal_conv1d_update(x, w, st, idxs[i % 4])

    # a ~12 us launch: the per-step events would add several microseconds to
    # each step, so the kernel time is the mean of a back-to-back pass
    tm = _time_gpu(step, steps, warmup, back_to_back=True)
    ms, kern_ms = tm.step_ms, tm.back_to_back_ms
    nbytes = 4 * B * D + 2 * D * W + 2 * B * (W - 1) * D * 4
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    return {"batch": B, "ms_per_step": ms, "kernel_ms": kern_ms, "kernel_ms_per_step_events": tm.median_ms,
            "kernel_ms_mean": tm.mean_ms, "GB_per_s": gbs,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "traffic": _traffic("causal_conv1d_step_kernel"),
                         "bytes_per_launch": nbytes, "kernel": "causal_conv1d_step_kernel"}}


def bench_decode_fused(dev, steps, warmup, cpu_budget):
    """Fused decode step (conv update + L2 norm + gating + recurrent step), and
    the same step as the separate ops in the reference's dtype flow."""
    import torch.nn.functional as F

    from myvllm_amd import causal_conv1d_update, gated_delta_net_decode_step, recurrent_gated_delta_rule
    from myvllm_amd.workloads import CONV_WIDTH, decode_fused_case

    B, slots = 256, 1024
    D = 2 * HK * DK + HV * DV
    case = decode_fused_case(B=B, num_slots=slots, seed=0, state=False)
    gen = torch.Generator(device=dev).manual_seed(0)
    state = torch.randn(slots, HV, DK, DV, device=dev, generator=gen) * 0.1
    perm = torch.randperm(slots, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    idxs = [perm[i * B:(i + 1) * B].to(dev) for i in range(4)]
    x, w, cs, a, b, A_log, dt_bias = (t.to(dev) for t in (case.mixed_qkv, case.conv_weight, case.conv_state, case.a,
                                                          case.b, case.A_log, case.dt_bias))

    def step(i):
        gated_delta_net_decode_step(x, w, cs, idxs[i % 4], a, b, A_log, dt_bias, state, idxs[i % 4], HK)

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms

    def separate(i):  # layers/linear_attention.py:89-90, :95, :97-114, :119 as separate ops
        beta = b.sigmoid()
        g = -A_log.float().exp() * F.softplus(a.float() + dt_bias)
        y = causal_conv1d_update(x, w, cs, idxs[i % 4])
        q, k, v = torch.split(y, [HK * DK, HK * DK, HV * DV], dim=-1)
        q, k, v = q.reshape(B, HK, DK), k.reshape(B, HK, DK), v.reshape(B, HV, DV)
        q = q * torch.rsqrt(q.pow(2).sum(dim=-1, keepdim=True) + 1e-6)
        k = k * torch.rsqrt(k.pow(2).sum(dim=-1, keepdim=True) + 1e-6)
        recurrent_gated_delta_rule(q, k, v, g, beta, state, idxs[i % 4])

    ms_sep = _time_gpu(separate, steps, warmup).step_ms
    per_seq = 2 * HV * DK * DV * 4 + 2 * (CONV_WIDTH - 1) * D * 4 + D * 2 + HV * DV * 2 + 2 * HV * 2
    nbytes = per_seq * B + D * CONV_WIDTH * 2 + 2 * HV * 4
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    return {"batch": B, "ms_per_step": ms, "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms, "GB_per_s": gbs,
            "separate_ops_ms_per_step": ms_sep,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "traffic": _traffic("gdn_decode_fused_kernel"),
                         "bytes_per_launch": nbytes, "kernel": "gdn_decode_fused_kernel"}}


def bench_layer(dev, steps, warmup, cpu_budget):
    """The full GDN layer (hidden 2048, Hk 16 / Hv 32, d 128) on a mixed batch of
    4 x 2048 prefill tokens and 128 decode tokens, with a per-stage breakdown."""
    from myvllm_amd import causal_conv1d_fn, chunk_gated_delta_rule, gated_delta_net_decode_step
    from myvllm_amd.cache import LinearAttentionCache
    from myvllm_amd.layer import GatedDeltaNet
    from myvllm_amd.norm import gdn_gating, rms_norm_gated
    from myvllm_amd.workloads import cu_from_lengths

    hidden, n_pre, len_pre, n_dec = 2048, 4, 2048, 128
    layer = GatedDeltaNet(hidden, HK, HV, DK, DV, device=dev)
    layer.init_random(std=0.02, seed=0)
    cache = LinearAttentionCache(1, n_pre + n_dec, 4, DK, DV, HK, HV, torch.bfloat16, dev, conv_dtype=torch.float32)
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    slots = torch.tensor([cache.allocate() for _ in range(n_pre + n_dec)], dtype=torch.int32, device=dev)
    T = n_pre * len_pre + n_dec
    x = torch.randn(T, hidden, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(dev)
    cu = cu_from_lengths([len_pre] * n_pre).to(dev)

    def step(_):
        layer(x, cu, slots, slots, num_decode_tokens=n_dec)

    ms = _time_gpu(step, steps, warmup).step_ms

    # the same forward, stage by stage, with events between the stages
    Tp, Np, L = n_pre * len_pre, n_pre, layer
    names = ["in_proj GEMM", "conv + q/k L2 norm", "gating", "chunked prefill", "fused decode step",
             "gated RMSNorm", "out_proj GEMM"]
    cz = L.conv_dim + L.v_size
    acc = [0.0] * len(names)
    stream = torch.cuda.current_stream()
    for it in range(warmup + steps):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
        ev[0].record(stream)
        proj = x @ L.in_proj.t()
        ev[1].record(stream)
        qkv, z = proj[:, :L.conv_dim], proj[:, L.conv_dim:cz]
        b, a = proj[:, cz:cz + HV], proj[:, cz + HV:]
        y = causal_conv1d_fn(qkv[:Tp], L.conv1d_weight, L.conv_state, slots[:Np], cu, l2norm_channels=2 * L.k_size)
        ev[2].record(stream)
        g, beta = gdn_gating(a[:Tp], b[:Tp], L.A_log, L.dt_bias)
        ev[3].record(stream)
        o = torch.empty(T, HV, DV, dtype=x.dtype, device=dev)
        chunk_gated_delta_rule(y[:, :L.k_size].view(Tp, HK, DK), y[:, L.k_size:2 * L.k_size].view(Tp, HK, DK),
                               y[:, 2 * L.k_size:].view(Tp, HV, DV), g, beta, L.recurrent_state, slots[:Np], cu,
                               out=o[:Tp])
        ev[4].record(stream)
        gated_delta_net_decode_step(qkv[Tp:], L.conv1d_weight, L.conv_state, slots[Np:], a[Tp:], b[Tp:], L.A_log,
                                    L.dt_bias, L.recurrent_state, slots[Np:], HK, out=o[Tp:])
        ev[5].record(stream)
        on = rms_norm_gated(o, z.view(T, HV, DV), L.norm_weight, L.rms_norm_eps)
        ev[6].record(stream)
        on.view(T, L.v_size) @ L.out_proj.t()
        ev[7].record(stream)
        torch.cuda.synchronize()
        if it >= warmup:
            for i in range(len(names)):
                acc[i] += ev[i].elapsed_time(ev[i + 1]) / steps
    gemm_flop = 2 * T * hidden * (L.conv_dim + L.v_size + 2 * HV) + 2 * T * L.v_size * hidden
    gdn_flop = PREFILL_FLOP_PER_TOKEN * Tp
    flop = gemm_flop + gdn_flop
    achieved = flop / (ms * 1e-3) / 1e12
    return {"tokens": T, "prefill_tokens": Tp, "decode_tokens": n_dec, "ms_per_step": ms, "kernel_ms": ms, "kernel_ms_mean": ms,
            "tokens_per_s": T / (ms * 1e-3),
            "stages_ms": {n: round(v, 4) for n, v in zip(names, acc)},
            "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                         "frac": achieved / PEAK_MFMA_TFLOPS, "traffic": None, "flop_per_launch": flop,
                         "kernel": "whole layer (GEMMs + GDN prefill FLOPs over the step time)"}}


def bench_attn_prefill(dev, steps, warmup, cpu_budget):
    """Causal varlen attention prefill of the hybrid stack's attention layers
    (Hq 16, Hkv 2, D 256) over the GDN prefill workload's 16 sequence lengths."""
    from myvllm_amd import flash_attention_prefill
    from myvllm_amd.workloads import ATTN_D, ATTN_HKV, ATTN_HQ, attn_prefill_32k_case

    case = attn_prefill_32k_case()
    q, k, v, cu = (t.to(dev) for t in (case.q, case.k, case.v, case.cu))
    out = torch.empty_like(q)
    max_len = case.max_len

    def step(_):
        flash_attention_prefill(q, k, v, cu, case.scale, ATTN_HQ, ATTN_HKV, ATTN_D, ATTN_D, True,
                                max_seqlen=max_len, out=out)

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms
    lens = (case.cu[1:] - case.cu[:-1]).tolist()
    tokens = int(case.cu[-1])
    pairs = sum(n * (n + 1) // 2 for n in lens)  # (query, visible key) pairs
    flops = 4 * ATTN_D * ATTN_HQ * pairs  # QK^T and PV, 2 FLOPs per MAC
    tflops = flops / (kern_ms * 1e-3) / 1e12
    res = {
        "tokens": tokens,
        "ms_per_step": ms,
        "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms,
        "tokens_per_s": tokens / (kern_ms * 1e-3),
        "TFLOP_per_s": tflops,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / PEAK_MFMA_TFLOPS, "traffic": _traffic("attn_prefill_kernel"),
                     "flop_per_launch": flops, "kernel": "attn_prefill_kernel"},
    }
    if cpu_budget > 0:
        from oracle.attention import attention_rows_ref

        _cpu_setup()
        n0 = lens[2]  # bounded sample: the third sequence (1,405 tokens) in full
        s0 = int(case.cu[2])
        sl = slice(s0, s0 + n0)
        sec = _time_cpu(lambda: attention_rows_ref(case.q[sl], case.k[sl], case.v[sl], torch.arange(n0), case.scale),
                        cpu_budget, max_reps=3)
        res["cpu_baseline"] = _cpu_baseline(n0 / sec, "tokens/s", f"one sequence of {n0} tokens, fp64 causal attention")
    return res


def bench_attn_paged_prefill(dev, steps, warmup, cpu_budget):
    """Chunked prefill over a paged KV cache (16 sequences, cached prefixes
    U[0, 4096], new chunks U[256, 2048], 16-token pages, Hq 16 / Hkv 2, D 256)."""
    from myvllm_amd import paged_flash_attention_prefill
    from myvllm_amd.workloads import ATTN_D, ATTN_HQ, attn_paged_prefill_case

    case = attn_paged_prefill_case()
    q, kc, vc, tab, ctx, cu = (t.to(dev) for t in (case.q, case.k_cache, case.v_cache, case.block_tables,
                                                    case.context_lens, case.cu))
    out = torch.empty_like(q)
    max_len = case.max_len

    def step(_):
        paged_flash_attention_prefill(q, kc, vc, tab, ctx, cu, None, case.scale, case.page, max_seqlen=max_len,
                                      out=out)

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms
    lens = (case.cu[1:] - case.cu[:-1]).tolist()
    ctxs = case.context_lens.tolist()
    pairs = sum(n * (L - n) + n * (n + 1) // 2 for n, L in zip(lens, ctxs))  # visible (query, key) pairs
    flops = 4 * ATTN_D * ATTN_HQ * pairs
    tflops = flops / (kern_ms * 1e-3) / 1e12
    tokens = int(case.cu[-1])
    return {
        "tokens": tokens,
        "cached_keys": int(sum(ctxs)),
        "ms_per_step": ms,
        "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms,
        "tokens_per_s": tokens / (kern_ms * 1e-3),
        "TFLOP_per_s": tflops,
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": PEAK_MFMA_TFLOPS, "unit": "TFLOP/s",
                     "frac": tflops / PEAK_MFMA_TFLOPS, "traffic": _traffic("attn_paged_prefill_kernel"),
                     "flop_per_launch": flops, "kernel": "attn_prefill_kernel (paged)"},
    }


def bench_attn_decode(dev, steps, warmup, cpu_budget):
    """Paged decode of the attention layers: batch 256, contexts uniform in
    [512, 4096] (602,903 cached keys), 16-token pages, Hq 16, Hkv 2, D 256."""
    from myvllm_amd import paged_flash_attention_decode
    from myvllm_amd.full_attention import decode_num_splits
    from myvllm_amd.workloads import ATTN_D, ATTN_HKV, ATTN_HQ, attn_decode_case

    case = attn_decode_case()
    q, kc, vc, tab, ctx = (t.to(dev) for t in (case.q, case.k_cache, case.v_cache, case.block_tables,
                                                case.context_lens))
    out = torch.empty_like(q)
    B = q.shape[0]
    splits = decode_num_splits(B, ATTN_HQ, ATTN_HKV, case.block_tables.shape[1] * case.page)

    def step(_):
        paged_flash_attention_decode(q, kc, vc, tab, ctx, case.scale, case.page, num_splits=splits, out=out)

    tm = _time_gpu(step, steps, warmup)
    ms, kern_ms = tm.step_ms, tm.median_ms
    keys = int(case.context_lens.sum())
    pages = int(((case.context_lens + case.page - 1) // case.page).sum())
    # K and V rows of every cached key, q and o, the table entries and lengths
    nbytes = keys * ATTN_HKV * ATTN_D * 2 * 2 + 2 * B * ATTN_HQ * ATTN_D * 2 + pages * 4 + B * 4
    gbs = nbytes / (kern_ms * 1e-3) / 1e9
    res = {
        "batch": B,
        "cached_keys": keys,
        "splits": splits,
        "ms_per_step": ms,
        "kernel_ms": kern_ms, "kernel_ms_mean": tm.mean_ms,
        "GB_per_s": gbs,
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                     "traffic": _traffic("attn_decode_kernel"), "bytes_per_launch": nbytes,
                     "kernel": "attn_decode_kernel + attn_decode_combine_kernel"},
    }
    if cpu_budget > 0:
        from oracle.attention import attention_rows_ref, gather_paged

        _cpu_setup()
        sub = 16  # bounded sample: 16 of the 256 sequences

        def cpu():
            for b in range(sub):
                L = int(case.context_lens[b])
                attention_rows_ref(case.q[b:b + 1], gather_paged(case.k_cache, case.block_tables[b], L),
                                   gather_paged(case.v_cache, case.block_tables[b], L), [L - 1], case.scale)

        sec = _time_cpu(cpu, cpu_budget, max_reps=3)
        sub_bytes = int(case.context_lens[:sub].sum()) * ATTN_HKV * ATTN_D * 2 * 2
        res["cpu_baseline"] = _cpu_baseline(sub_bytes / sec / 1e9, "GB/s",
                                            f"{sub} of {B} sequences, fp64 attention over gathered pages")
    return res


def _hbm_copy_fn(src, dst, blocks):
    from myvllm_amd import _lib

    lib = _lib.load()
    stream = _lib.stream_handle(src.device)

    def step(_):
        _lib.check("gdn_hbm_copy", lib.gdn_hbm_copy(src.data_ptr(), dst.data_ptr(), src.numel(), blocks, stream))

    return step


HBM_COPY_BLOCKS = (1024, 2048, 4096, 8192, 0)  # grids the ceiling is taken over (0: one pass, 262,144 workgroups)


def bench_hbm_copy(dev, steps, warmup, cpu_budget, blocks=None):
    """Plain 1 GiB device-to-device copy with the library's HIP streaming
    kernel (16-byte non-temporal loads and stores): the calibration point of
    the HBM byte counters and the measured bandwidth ceiling of this device.
    Without ``blocks`` the best of the grids in HBM_COPY_BLOCKS is reported."""
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).random_()
    dst = torch.empty_like(src)
    best = None
    for nb in ((blocks,) if blocks is not None else HBM_COPY_BLOCKS):
        tm = _time_gpu(_hbm_copy_fn(src, dst, nb), steps, warmup)
        if best is None or tm.median_ms < best[1].median_ms:
            best = (nb, tm)
    assert torch.equal(src[-4096:], dst[-4096:]) and torch.equal(src[:4096], dst[:4096])
    nb, tm = best
    nbytes = 2 * n
    gbs = nbytes / (tm.median_ms * 1e-3) / 1e9
    return {"bytes": nbytes, "blocks": nb, **tm.fields(), "GB_per_s": gbs,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": gbs / PEAK_HBM_GBS, "traffic": None, "bytes_per_launch": nbytes,
                         "kernel": "hbm_stream_copy_kernel"}}


def measure_peaks(dev, steps, warmup):
    """Ceilings measured on this device beside the datasheet peaks: a large
    bf16 GEMM through torch (hipBLASLt) and a 1 GiB streaming copy (the
    library's plain HIP copy kernel, best grid; torch's copy_ beside it)."""
    n = 8192
    gen = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=gen)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=gen)
    c = torch.empty(n, n, device=dev, dtype=torch.bfloat16)
    kern_ms = _time_gpu(lambda _: torch.matmul(a, b, out=c), steps, warmup).median_ms
    gemm = 2 * n ** 3 / (kern_ms * 1e-3) / 1e12
    del a, b, c
    stream = bench_hbm_copy(dev, steps, warmup, 0)
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch_ms = _time_gpu(lambda _: dst.copy_(src), steps, warmup).median_ms
    return {"gemm_bf16_TFLOP_per_s": gemm, "gemm": f"torch.matmul bf16 {n}x{n}x{n} (hipBLASLt)",
            "stream_GB_per_s": stream["GB_per_s"],
            "stream": "hbm_stream_copy_kernel, 1 GiB, " + (f"{stream['blocks']} workgroups" if stream["blocks"] else
                                                           "one pass of 262,144 workgroups") + " (read + write counted)",
            "torch_copy_GB_per_s": 2 * (1 << 30) / (torch_ms * 1e-3) / 1e9}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="all",
                    help="all, or a comma-separated list of prefill, prefill_short, prefill_skewed, decode, conv, "
                         "conv_update, "
                         "decode_fused, "
                         "layer, attn_prefill, attn_paged_prefill, attn_decode, hbm_copy")
    ap.add_argument("--settle-ms", type=float, default=300.0,
                    help="untimed run of each workload before its warm-up steps, in ms of wall time (0 disables it)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="time budget of each CPU-oracle baseline (0 disables it)")
    ap.add_argument("--copy-blocks", type=int, default=None,
                    help="hbm_copy workload: one grid size (workgroups; 0 = one pass) instead of the sweep")
    args = ap.parse_args()
    if args.steps < 1 or args.warmup < 0 or args.settle_ms < 0:
        ap.error("--steps must be at least 1, --warmup and --settle-ms at least 0")
    global SETTLE_MS
    SETTLE_MS = args.settle_ms
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the GDN path is benchmarked on a single MI355X "
              "(the kernels shard over heads and sequences with no communication inside the ops, so each "
              "GPU would run them on its share). "
              "Run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    known = {"prefill", "prefill_short", "prefill_skewed", "decode", "conv", "conv_update", "decode_fused", "layer",
             "attn_prefill", "attn_paged_prefill", "attn_decode", "hbm_copy"}
    chosen = set(args.workload.split(","))
    if not chosen <= (known | {"all"}):
        print(f"unknown workload(s): {sorted(chosen - known - {'all'})}", file=sys.stderr)
        sys.exit(2)
    parts = {}
    want = (lambda w: "all" in chosen or w in chosen)
    if want("prefill"):
        parts["prefill"] = bench_prefill(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# prefill: {parts['prefill']['kernel_ms'] * 1e3:.1f} us/launch", file=sys.stderr, flush=True)
    if want("prefill_short"):
        parts["prefill_short"] = bench_prefill_short(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# prefill_short: {parts['prefill_short']['kernel_ms'] * 1e3:.1f} us/launch "
              f"({parts['prefill_short']['roofline']['achieved']:.0f} GB/s)", file=sys.stderr, flush=True)
    if "prefill_skewed" in chosen:  # (named explicitly only: it shares the short-sequence kernel)
        parts["prefill_skewed"] = bench_prefill_skewed(dev, min(args.steps, 20), min(args.warmup, 5), args.cpu_seconds)
        print(f"# prefill_skewed: {parts['prefill_skewed']['kernel_ms'] * 1e3:.1f} us/launch (one item per "
              f"workgroup: {parts['prefill_skewed']['one_item_per_workgroup_kernel_ms'] * 1e3:.1f})",
              file=sys.stderr, flush=True)
    if want("decode"):
        parts["decode"] = bench_decode(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# decode: {parts['decode']['kernel_ms'] * 1e3:.1f} us/launch", file=sys.stderr, flush=True)
    if want("conv"):
        parts["conv"] = bench_conv(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# conv: {parts['conv']['kernel_ms'] * 1e3:.1f} us/launch", file=sys.stderr, flush=True)
    if want("conv_update"):
        parts["conv_update"] = bench_conv_update(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# conv_update: {parts['conv_update']['kernel_ms'] * 1e3:.1f} us/launch", file=sys.stderr, flush=True)
    if want("decode_fused"):
        parts["decode_fused"] = bench_decode_fused(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# decode_fused: {parts['decode_fused']['kernel_ms'] * 1e3:.1f} us/launch "
              f"(separate ops: {parts['decode_fused']['separate_ops_ms_per_step'] * 1e3:.1f} us/step)",
              file=sys.stderr, flush=True)
    if want("layer"):
        parts["layer"] = bench_layer(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# layer: {parts['layer']['ms_per_step'] * 1e3:.1f} us/step "
              f"({parts['layer']['tokens_per_s'] / 1e6:.2f} M tokens/s); stages (us): "
              + ", ".join(f"{k} {v * 1e3:.1f}" for k, v in parts["layer"]["stages_ms"].items()),
              file=sys.stderr, flush=True)
    if want("attn_prefill"):
        parts["attn_prefill"] = bench_attn_prefill(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# attn_prefill: {parts['attn_prefill']['kernel_ms'] * 1e3:.1f} us/launch "
              f"({parts['attn_prefill']['TFLOP_per_s']:.0f} TFLOP/s)", file=sys.stderr, flush=True)
    if want("attn_paged_prefill"):
        parts["attn_paged_prefill"] = bench_attn_paged_prefill(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# attn_paged_prefill: {parts['attn_paged_prefill']['kernel_ms'] * 1e3:.1f} us/launch "
              f"({parts['attn_paged_prefill']['TFLOP_per_s']:.0f} TFLOP/s)", file=sys.stderr, flush=True)
    if want("attn_decode"):
        parts["attn_decode"] = bench_attn_decode(dev, args.steps, args.warmup, args.cpu_seconds)
        print(f"# attn_decode: {parts['attn_decode']['kernel_ms'] * 1e3:.1f} us/step "
              f"({parts['attn_decode']['GB_per_s']:.0f} GB/s)", file=sys.stderr, flush=True)
    if "hbm_copy" in chosen:
        parts["hbm_copy"] = bench_hbm_copy(dev, args.steps, args.warmup, args.cpu_seconds, blocks=args.copy_blocks)
    peaks = None
    if "all" in chosen:
        # each MFMA-bound roofline also as a fraction of a measured library GEMM,
        # each HBM-bound one as a fraction of the measured streaming-copy rate
        peaks = measure_peaks(dev, min(args.steps, 20), min(args.warmup, 5))
        for part in parts.values():
            roof = part.get("roofline")
            if roof and roof["bound"] == "mfma":
                roof["frac_of_measured_gemm"] = roof["achieved"] / peaks["gemm_bf16_TFLOP_per_s"]
            elif roof and roof["bound"] == "hbm":
                roof["frac_of_measured_stream"] = roof["achieved"] / peaks["stream_GB_per_s"]
        print(f"# measured peaks: GEMM {peaks['gemm_bf16_TFLOP_per_s']:.0f} TFLOP/s, "
              f"stream copy {peaks['stream_GB_per_s']:.0f} GB/s (torch copy_ {peaks['torch_copy_GB_per_s']:.0f})",
              file=sys.stderr, flush=True)

    head_name = "prefill" if "prefill" in parts else next(iter(parts))
    head = parts.pop(head_name)
    if head_name == "prefill":
        metric, value, unit = "GDN prefill tokens/s", head["tokens_per_s"], "tokens/s"
        workload = (f"gdn_chunk_prefill: 16 varlen seqs (lengths U[512,4096], seed 0), {head['tokens']} tokens, "
                    f"Hk {HK} / Hv {HV}, d {DK}, chunk {CHUNK}, bf16 q/k/v, fp32 g/beta/state")
    elif head_name == "prefill_short":
        metric, value, unit = "GDN prefill tokens/s", head["tokens_per_s"], "tokens/s"
        workload = (f"gdn_chunk_prefill: {head['sequences']} sequences of 64 tokens ({head['tokens']} tokens), "
                    f"Hk {HK} / Hv {HV}, d {DK}, bf16 q/k/v, fp32 g/beta/state")
    elif head_name == "decode":
        metric, value, unit = "GDN decode state-update HBM GB/s", head["GB_per_s"], "GB/s"
        workload = "gdn_recurrent_step: batch 256 from a 1024-slot fp32 state cache, Hk 16 / Hv 32, d 128"
    elif head_name == "decode_fused":
        metric, value, unit = "GDN fused decode step HBM GB/s", head["GB_per_s"], "GB/s"
        workload = ("gdn_decode_step_fused: batch 256, conv update (8192 channels, width 4, fp32 conv state) + "
                    "L2 norm + gating + recurrent step from a 1024-slot fp32 state cache, Hk 16 / Hv 32, d 128")
    elif head_name == "layer":
        metric, value, unit = "GDN layer tokens/s", head["tokens_per_s"], "tokens/s"
        workload = ("GatedDeltaNet layer: hidden 2048, Hk 16 / Hv 32, d 128, conv 4; 4 x 2048 prefill + 128 decode "
                    "tokens in one call, bf16 weights ~N(0, 0.02), fp32 states")
    elif head_name == "attn_prefill":
        metric, value, unit = "attention prefill tokens/s", head["tokens_per_s"], "tokens/s"
        workload = (f"flash_attention_varlen: causal, 16 varlen seqs (lengths U[512,4096], seed 0), "
                    f"{head['tokens']} tokens, Hq 16 / Hkv 2, d 256, bf16")
    elif head_name == "attn_paged_prefill":
        metric, value, unit = "attention paged prefill tokens/s", head["tokens_per_s"], "tokens/s"
        workload = ("paged_attention_prefill: 16 seqs, cached prefixes U[0,4096], new chunks U[256,2048], "
                    "16-token pages, Hq 16 / Hkv 2, d 256, bf16")
    elif head_name == "attn_decode":
        metric, value, unit = "attention paged decode HBM GB/s", head["GB_per_s"], "GB/s"
        workload = ("paged_attention_decode: batch 256, contexts U[512,4096] (602,903 keys), 16-token pages, "
                    "Hq 16 / Hkv 2, d 256, bf16")
    elif head_name == "hbm_copy":
        metric, value, unit = "device copy HBM GB/s", head["GB_per_s"], "GB/s"
        workload = "hbm_copy: 1 GiB device-to-device copy (read + write counted)"
    else:
        metric, value, unit = f"causal_conv1d {head_name} HBM GB/s", head["GB_per_s"], "GB/s"
        workload = f"causal_conv1d {head_name}: 8192 channels, width 4, bf16 x/w, fp32 conv state"
    line = {
        "metric": metric,
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.Generator, CPU-drawn, copied to HBM before timing)",
        "config": {"workload": workload, "kernel_ms": head["kernel_ms"], "settle_ms": args.settle_ms},
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
    }
    if peaks is not None:
        line["measured_peaks"] = peaks
    for name, part in parts.items():
        line[name] = part
    print(json.dumps(line))


if __name__ == "__main__":
    main()
