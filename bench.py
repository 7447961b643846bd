"""Benchmark of the MI355X chunked GatedDeltaNet forward (BASELINE.json metric).

One step = one chunk_gated_delta_rule forward over BASELINE config 2
(B=1, T=32760, H=20, dk=dv=128, chunk 64, bf16 q/k/v/beta, fp32 g and h0,
output_final_state=True) with inputs resident in HBM, through the C ABI
(kairos_gdn_chunk_fwd).  Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu-baseline]
  python bench.py --config 1|3|4      # the other BASELINE configs (4: 21-frame fp8 rollout), one line each
  python bench.py --l2norm            # config 2 with use_qk_l2norm_in_kernel=True (the layer's own mode)
  python bench.py --calibrate-copy 1024     # reference copy kernel for rocprofv3 counter scaling
  python bench.py --epilogue                # the gated RMSNorm output epilogue on config 2's o
  python bench.py --model-shape             # the Kairos 4B layer's head dims dk=256, dv=512
  python bench.py --recurrent               # the short-sequence mode's decoding step (fused_recurrent)
  python bench.py --prologue                # the layer prologue: causal conv + SiLU (+ q/k L2 norm), gates

Timing (every mode): an untimed warm-up of at least --warmup steps AND at
least --warmup-seconds of wall time (so the timed steps run at steady clocks;
both figures are in the JSON), then exactly --steps steps between two device
synchronisations.  `value` and `ms_per_step` come from that wall-clock
interval; `step_ms` gives the median / p10 / p90 of per-step HIP events
recorded on the launch stream in the same loop.  `cold_step_ms` times steps
that each follow an overwrite of a 640 MiB buffer, which evicts the 256 MiB
Infinity Cache (MALL) and the L2s, so every input comes from HBM: a fixed 100 of
them (after 5 discarded), whatever --steps is, so runs of any length agree.

Roofline: `achieved` = the op's algorithmic HBM bytes (the fused minimum:
q, k, v and o once, 2*dk*s_qk + 4*dv + 8 bytes per token-head plus the initial and final
state, 678.8 MB at config 2) over the dominant kernel's average duration;
`whole_call` puts the same bytes over the median step.  `design_bytes` is what
this design's dominant kernel must move (its inputs include the chunk records and
segment states of the fused path).  `traffic` is the whole call's measured HBM
bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE summed over the call's kernels, from
the committed summary in profiles/), `traffic_kernel` the dominant kernel's.
"""
import argparse
import ctypes
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kairos-sensenova_amd"))

import torch  # noqa: E402

METRIC = "GDN chunk-fwd tokens/s + TFLOP/s (% bf16 MFMA peak) at T=32760,H=20,d=128"
PEAK_BF16_TFLOPS = 2516.6      # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
C = 64
RECORD = C * C * 2 + 8 * C * 4      # bytes of one (chunk, head) record written by seg_prep
KERNELS = ["seg_prep_kernel", "seg_trans_kernel", "seg_combine_kernel", "seg_out_kernel"]
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "chunk_fwd_config2.md")
MODEL_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "chunk_fwd_model_shape.md")
MODEL_L2_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "chunk_fwd_model_shape_l2norm.md")
FLUSH_BYTES = 640 << 20
COLD_STEPS = 100           # cold (flushed) steps timed in every mode, whatever --steps is
COLD_DISCARD = 5          # cold steps run first and not counted

# BASELINE.json configs measured here (config 0 is the CPU plumbing case, a parity test only)
CONFIGS = {
    1: dict(B=1, T=8192, H=20, K=128, V=128, cu=None, seed=20261),
    2: dict(B=1, T=32760, H=20, K=128, V=128, cu=None, seed=20262),
    3: dict(B=1, T=53040, H=20, K=128, V=128, cu=[0, 1560, 7800, 20280, 53040], seed=20263),
    4: dict(B=8, T=1560, H=20, K=128, V=128, cu=None, seed=20264, frames=21),
}


def flops_per_tok_head(K, V):
    """Algorithmic FLOPs per (token, head), every MMA tile counted at full size."""
    return 6 * K * V + 6 * C * K + 4 * C * V


def alg_bytes(tok_heads, n_states, K, V, s_qk=2, s_v=2):
    """The op's algorithmic (compulsory) HBM bytes, the fused minimum: q, k, v, o once per
    token-head plus 8 bytes for the gate and beta, and the initial state read and the final state
    written (fp32) per (sequence, head): 1,032 B per token-head + 128 KiB per (sequence, head) at d=128."""
    return tok_heads * (2 * K * s_qk + 2 * V * s_v + 8) + n_states * 2 * K * V * 4


def kernel_models(B, T, H, K, V, L, s=2, s_g=4, s_b=2):
    """Design HBM bytes (what each kernel of this design reads and writes) and FLOPs of one launch.

    seg_prep reads k, g, beta and writes one chunk record per (chunk, head):
    the bf16 inverse Ai (64 x 64) and eight fp32 vectors of 64, RECORD bytes.
    seg_out reads q, k, v, the records and the segment initial states, writes
    o and final_state; seg_trans reads k, v and the records of every segment
    but the last of each sequence and writes its [M | R]; seg_combine reads
    [M | R] and h0 and writes the segment initial states.  FLOPs count every
    MMA tile at full size.
    """
    nc = (T + C - 1) // C
    nseg = (nc + L - 1) // L
    tok = B * T * H
    tok_trans = B * H * min(T, (nseg - 1) * L * C)
    rec_trans = B * H * min(nc, (nseg - 1) * L) * RECORD
    state = K * V * 4
    mr = (K * K + K * V) * 4
    return {
        "seg_prep_kernel": dict(
            bytes=tok * (K * s + s_g + s_b) + B * H * nc * RECORD,
            flops=tok * 2 * C * K),
        "seg_trans_kernel": dict(
            bytes=tok_trans * (K * s + V * s) + rec_trans + B * H * (nseg - 1) * mr,
            flops=tok_trans * (2 * C * (K + V) + 4 * K * (K + V))),
        "seg_combine_kernel": dict(
            bytes=B * H * (nseg - 1) * (mr + state) + B * H * state,
            flops=B * H * (nseg - 1) * 2 * K * K * V),
        "seg_out_kernel": dict(
            bytes=tok * (2 * K * s + V * s + V * s) + B * H * nc * RECORD + B * H * (nseg - 1) * state
            + 2 * B * H * state,
            flops=tok * (flops_per_tok_head(K, V) - 2 * C * K)),
    }


def measured_traffic():
    """{kernel: HBM bytes per launch} from the committed rocprofv3 summary (empty if absent)."""
    out = {}
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                m = re.match(r"\s*traffic_bytes_per_launch\s+(\S+)\s+(\d+)", ln)
                if m:
                    out[m.group(1)] = int(m.group(2))
    except OSError:
        pass
    return out


def measured_call_traffic(path, name):
    """HBM bytes per call of the workload `name` from a committed rocprofv3 summary (None if absent)."""
    try:
        with open(path) as f:
            for ln in f:
                m = re.match(r"\s*traffic_bytes_per_call\s+(\S+)\s+(\d+)", ln)
                if m and m.group(1) == name:
                    return int(m.group(2))
    except OSError:
        pass
    return None


def pct(xs, p):
    """p-th percentile (linear interpolation) of a non-empty list."""
    s = sorted(xs)
    i = (len(s) - 1) * p / 100.0
    lo = int(math.floor(i))
    hi = min(lo + 1, len(s) - 1)
    return s[lo] + (s[hi] - s[lo]) * (i - lo)


def summary(xs):
    return {"median": statistics.median(xs), "p10": pct(xs, 10), "p90": pct(xs, 90), "mean": statistics.fmean(xs),
            "n": len(xs)}


class Timer:
    """Steady-state timing of a step function on the current stream (see the module docstring)."""

    def __init__(self, args):
        self.steps, self.warmup, self.floor = args.steps, args.warmup, args.warmup_seconds
        # cold steps: a fixed count, whatever --steps is, after a few discarded ones (the first flushes
        # change the clocks), so that runs of any length report the same measurement
        self.cold_steps = 0 if args.no_cold else COLD_STEPS
        self.cold_discard = COLD_DISCARD

    def warm(self, step):
        t0 = time.perf_counter()
        n = 0
        while n < self.warmup or time.perf_counter() - t0 < self.floor:
            for _ in range(10):           # bounded queue: synchronise every 10 steps
                step()
                n += 1
            torch.cuda.synchronize()
        return n, time.perf_counter() - t0

    def run(self, step):
        n_warm, t_warm = self.warm(step)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(self.steps + 1)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev[0].record()
        for i in range(self.steps):
            step()
            ev[i + 1].record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / self.steps
        hot = [ev[i].elapsed_time(ev[i + 1]) for i in range(self.steps)]
        res = {"wall_s": wall, "step_ms": summary(hot), "warmup_steps_run": n_warm, "warmup_wall_s": t_warm}
        if self.cold_steps:
            flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device="cuda")
            n = self.cold_discard + self.cold_steps
            e0 = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
            e1 = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
            for i in range(n):
                flush.fill_(i & 0xFF)
                e0[i].record()
                step()
                e1[i].record()
            torch.cuda.synchronize()
            res["cold_step_ms"] = summary([a.elapsed_time(b) for a, b in zip(e0, e1)][self.cold_discard:])
            del flush
        return res

    def fields(self, res):
        out = {"step_ms": res["step_ms"], "warmup_steps_run": res["warmup_steps_run"],
               "warmup_wall_s": round(res["warmup_wall_s"], 3), "warmup_floor_s": self.floor}
        if "cold_step_ms" in res:
            out["cold_step_ms"] = res["cold_step_ms"]
            out["cold_flush_bytes"] = FLUSH_BYTES
        return out


# ---------------------------------------------------------------------------
# inputs
# ---------------------------------------------------------------------------
def make_inputs(B, T, H, K, V, seed, n_states=None, device="cpu", dtype=torch.bfloat16):
    """BASELINE distributions: q, k ~ N(0,1) then L2-normalised per head; v ~ N(0,1); beta = sigmoid(N(0,1));
    g = -softplus(N(0,1)) fp32; h0 = 0.02 N(0,1) fp32 ([n_states or B, H, K, V])."""
    g_ = torch.Generator(device="cpu").manual_seed(seed)

    def unit(shape):
        return torch.nn.functional.normalize(torch.randn(shape, generator=g_), dim=-1)
    q = unit((B, T, H, K)).to(device, dtype)
    k = unit((B, T, H, K)).to(device, dtype)
    v = torch.randn((B, T, H, V), generator=g_).to(device, dtype)
    beta = torch.sigmoid(torch.randn((B, T, H), generator=g_)).to(device, dtype)
    g = (-torch.nn.functional.softplus(torch.randn((B, T, H), generator=g_))).to(device, torch.float32)
    h0 = (0.02 * torch.randn((n_states or B, H, K, V), generator=g_)).to(device, torch.float32)
    return q, k, v, g, beta, h0


def quantize_fp8(x):
    """Per-head e4m3 quantisation of [B, T, H, K] with scale = amax / 448."""
    xf = x.float()
    scale = (xf.abs().amax(dim=(0, 1, 3)) / 448.0).clamp_min(1e-12)
    codes = (xf / scale[None, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return codes, scale


# ---------------------------------------------------------------------------
# CPU baseline: the fp32 torch-CPU restatement on the host cores available to this job
# ---------------------------------------------------------------------------
def host_threads():
    """Threads for the CPU leg: the CPUs this process may run on, capped by a cgroup CPU quota."""
    n_aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                quota = max(1, int(int(q) / int(period)))
    except (OSError, ValueError):
        pass
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    threads = n_aff if quota is None else min(n_aff, quota)
    return threads, {"os_cpu_count": os.cpu_count(), "affinity": n_aff, "cgroup_quota_cpus": quota, "model": model}


def cpu_baseline(B, T, H, K, V, cu, seed, tokens_per_run, label, min_seconds=10.0, max_runs=10):
    """Time oracle/gdn_torch_cpu.py (fp32 chunked restatement, torch-CPU batched matmuls) on the workload's
    own shape, repeated until min_seconds of CPU work (at most max_runs); rate = tokens_per_run / median."""
    sys.path.insert(0, ROOT)
    from oracle import gdn_torch_cpu as TC
    threads, info = host_threads()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        N = len(cu) - 1 if cu else B
        q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, seed, n_states=N, dtype=torch.float32)
        times = []
        t_start = time.perf_counter()
        while not times or (time.perf_counter() - t_start < min_seconds and len(times) < max_runs):
            t0 = time.perf_counter()
            TC.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, cu_seqlens=cu)
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    dt = statistics.median(times)
    return {"value": tokens_per_run / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle/gdn_torch_cpu.py fp32 chunked forward on {label} (all heads), {len(times)} runs in "
                      f"{sum(times):.1f} s, median {dt:.3f} s per run, torch.set_num_threads({threads}); host: "
                      f"{info['model']}; os.cpu_count()={info['os_cpu_count']}, affinity={info['affinity']}, "
                      f"cgroup quota={info['cgroup_quota_cpus']}"}


# ---------------------------------------------------------------------------
# the headline op (configs 1-3, optionally with the in-op L2 norm)
# ---------------------------------------------------------------------------
def bench_chunk(args, dev, cfg_id):
    from kairos_gdn import _lib
    cfg = CONFIGS[cfg_id]
    B, T, H, K, V, cu = cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], cfg["cu"]
    N = len(cu) - 1 if cu else B
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, cfg["seed"], n_states=N, device=dev)
    l2 = int(bool(args.l2norm))
    if l2:          # the layer hands the op unnormalised q, k (the op normalises them)
        q = (q.float() * 3.0).to(torch.bfloat16)
        k = (k.float() * 0.5).to(torch.bfloat16)
    scale = K ** -0.5
    lib = _lib.load()
    n_seqs = N if cu else 0
    cu_t = torch.tensor(cu, dtype=torch.int64, device=dev) if cu else None
    ws_bytes = lib.kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, n_seqs, _lib.BF16, _lib.BF16, l2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    ht = torch.empty(N, H, K, V, dtype=torch.float32, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_chunk_fwd", P(q), P(k), P(v), P(g), P(beta), None, None, P(h0), P(o), P(ht), P(cu_t),
                  n_seqs, B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, scale, l2, P(ws),
                  ws_bytes, sp)

    timer = Timer(args)
    res = timer.run(step)
    wall = res["wall_s"]

    # per-kernel times: hipEvents recorded by the library on the launch stream around each kernel
    lib.kairos_gdn_profile_begin()
    for _ in range(args.steps):
        step()
    avg = (ctypes.c_double * len(KERNELS))()
    ncalls = lib.kairos_gdn_profile_end(avg, len(KERNELS))
    if ncalls != args.steps:
        raise RuntimeError(f"kernel timing recorded {ncalls} calls: {lib.kairos_gdn_last_error().decode()}")
    per = {n: avg[i] for i, n in enumerate(KERNELS)}

    tok_heads = B * T * H
    alg = alg_bytes(tok_heads, N * H, K, V)
    flops = tok_heads * flops_per_tok_head(K, V)
    L = lib.kairos_gdn_segment_chunks(B, T, H, n_seqs)
    dom = max(KERNELS, key=lambda n: per[n])
    dom_s = per[dom] / 1e3
    med_s = res["step_ms"]["median"] / 1e3
    roof = {"bound": "hbm", "kernel": dom, "achieved": alg / dom_s / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": alg / dom_s / 1e9 / PEAK_HBM_GBS, "alg_bytes": alg,
            "whole_call": {"achieved": alg / med_s / 1e9, "frac": alg / med_s / 1e9 / PEAK_HBM_GBS},
            "traffic": None}
    if cfg_id == 2 and not l2 and cu is None:
        models = kernel_models(B, T, H, K, V, L)
        roof["design_bytes"] = models[dom]["bytes"]
        meas = measured_traffic()
        if all(n in meas for n in KERNELS):
            roof["traffic"] = sum(meas[n] for n in KERNELS)
            roof["traffic_scope"] = "whole call: " + " + ".join(KERNELS)
            roof["traffic_kernel"] = meas[dom]
            roof["traffic_over_alg"] = roof["traffic"] / alg
    name = {1: "BASELINE config 1", 2: "BASELINE config 2", 3: "BASELINE config 3 (varlen)"}[cfg_id]
    out = {
        "metric": METRIC if (cfg_id == 2 and not l2) else
        f"GDN chunk-fwd tokens/s + TFLOP/s at {name}" + (" with use_qk_l2norm_in_kernel=True" if l2 else ""),
        "value": B * T / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{name}: chunk_gated_delta_rule fwd B={B} T={T} H={H} dk=dv={K} chunk 64, bf16 "
                               "q/k/v/beta, fp32 g/h0, output_final_state, inputs resident in HBM"
                               + (f", cu_seqlens={cu}" if cu else "")
                               + (", use_qk_l2norm_in_kernel=True (unnormalised q, k)" if l2 else ""),
                   "segments_chunks": L},
        **timer.fields(res),
        "tflops": flops / wall / 1e12,
        "mfma_peak_frac": flops / wall / 1e12 / PEAK_BF16_TFLOPS,
        "tflops_median_step": flops / med_s / 1e12,
        "hbm_gbs_whole_op": alg / wall / 1e9,
        "kernels_ms": per,
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(B, T, H, K, V, cu, cfg["seed"], B * T, f"the full {name} workload")
    print(json.dumps(out), flush=True)


def bench_streaming(args, dev):
    """B=8, H=20, dk=dv=128; 21 sequential calls of T=1560 with the fp32 state carried,
    q/k fp8 e4m3 with per-head scales (amax / 448), v/beta bf16, g fp32.  A step is one 21-frame rollout;
    per-frame latency from HIP events around each call.  Drift: the streamed end state against one fp32 call
    over all 21 frames with the unquantised q/k and the rollout's own v, beta, g (this library's fp32 path,
    itself checked against the oracle by the tests)."""
    from kairos_gdn import _lib
    cfg = CONFIGS[4]
    B, Tf, H, K, V, F = cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"], cfg["frames"]
    frames = []
    for f in range(F):
        q, k, v, g, beta, _ = make_inputs(B, Tf, H, K, V, cfg["seed"] * 100 + f, device="cpu", dtype=torch.float32)
        qc, qs = quantize_fp8(q)
        kc, ks = quantize_fp8(k)
        frames.append(dict(q8=qc.to(dev), k8=kc.to(dev), qs=qs.to(dev), ks=ks.to(dev), v=v.to(dev, torch.bfloat16),
                           g=g.to(dev), beta=beta.to(dev, torch.bfloat16), qf=q, kf=k))
    h0 = (0.02 * torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(cfg["seed"]))).to(dev)
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_fwd_workspace_size(B, Tf, H, K, V, 0, _lib.F8E4M3, _lib.BF16, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    o = torch.empty(B, Tf, H, V, dtype=torch.bfloat16, device=dev)
    states = [torch.empty(B, H, K, V, dtype=torch.float32, device=dev) for _ in range(2)]
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731
    frame_ev = []

    def call(fr, s_in, s_out):
        _lib.call("kairos_gdn_chunk_fwd", P(fr["q8"]), P(fr["k8"]), P(fr["v"]), P(fr["g"]), P(fr["beta"]),
                  P(fr["qs"]), P(fr["ks"]), P(s_in), P(o), P(s_out), None, 0, B, Tf, H, K, V, _lib.F8E4M3, _lib.BF16,
                  _lib.F32, _lib.BF16, _lib.F32, K ** -0.5, 0, P(ws), ws_bytes, sp)

    def step(record=None):
        s_in = h0
        for f, fr in enumerate(frames):
            s_out = states[f % 2]
            if record is not None:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                call(fr, s_in, s_out)
                e1.record()
                record.append((e0, e1))
            else:
                call(fr, s_in, s_out)
            s_in = s_out
        return s_in

    timer = Timer(args)
    res = timer.run(step)
    wall = res["wall_s"]
    for _ in range(args.steps):
        step(frame_ev)
    torch.cuda.synchronize()
    per_frame = [a.elapsed_time(b) for a, b in frame_ev]
    end = step().clone()
    torch.cuda.synchronize()

    # single fp32 call over all frames, unquantised q/k
    cat = lambda key: torch.cat([fr[key] for fr in frames], dim=1).to(dev).contiguous()  # noqa: E731
    qf, kf, gf = cat("qf"), cat("kf"), cat("g")
    vf, bf = cat("v").float(), cat("beta").float()      # the same bf16 values the rollout reads
    T_all = Tf * F
    ws32_bytes = lib.kairos_gdn_chunk_fwd_workspace_size(B, T_all, H, K, V, 0, _lib.F32, _lib.F32, 0)
    ws32 = torch.empty(max(ws32_bytes, 1), dtype=torch.uint8, device=dev)
    o32 = torch.empty(B, T_all, H, V, dtype=torch.float32, device=dev)
    ref = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    _lib.call("kairos_gdn_chunk_fwd", P(qf), P(kf), P(vf), P(gf), P(bf), None, None, P(h0), P(o32), P(ref), None, 0,
              B, T_all, H, K, V, _lib.F32, _lib.F32, _lib.F32, _lib.F32, _lib.F32, K ** -0.5, 0, P(ws32), ws32_bytes,
              sp)
    torch.cuda.synchronize()
    drift = (torch.linalg.vector_norm(end - ref) / torch.linalg.vector_norm(ref)).item()
    del ws32, o32

    tok_heads = B * Tf * H
    alg = alg_bytes(tok_heads, B * H, K, V, s_qk=1)
    flops = tok_heads * flops_per_tok_head(K, V)
    fs = summary(per_frame)
    med_s = fs["median"] / 1e3
    out = {
        "metric": "GDN chunk-fwd streaming rollout (BASELINE config 4): tokens/s and per-frame latency",
        "value": B * Tf * F / wall, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": wall * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"BASELINE config 4: {F} sequential chunk_gated_delta_rule calls of B={B} T={Tf} H={H} "
                               f"dk=dv={K}, fp8 e4m3 q/k with per-head scales, bf16 v/beta, fp32 g, fp32 state "
                               "carried between calls; a step is one rollout",
                   "segments_chunks": lib.kairos_gdn_segment_chunks(B, Tf, H, 0)},
        **timer.fields(res),
        "frame_ms": fs,
        "frame_tflops_median": flops / med_s / 1e12,
        "end_state_drift_rel_l2": drift,
        "drift_reference": "one fp32 call over all 21 frames (T=32760) with unquantised q/k, same h0",
        "roofline": {"bound": "hbm", "kernel": "whole call (median frame)", "achieved": alg / med_s / 1e9,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": alg / med_s / 1e9 / PEAK_HBM_GBS,
                     "alg_bytes": alg, "traffic": None},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(B, Tf, H, K, V, None, cfg["seed"], B * Tf,
                                           f"one frame of config 4 (B={B}, T={Tf})")
    print(json.dumps(out), flush=True)


# ---------------------------------------------------------------------------
# backward (chunk.py:70-146 + the autograd backward, chunk.py:188-213)
# ---------------------------------------------------------------------------
def bwd_flops_per_tok_head(K, V):
    """Algorithmic FLOPs of the reference backward per (token, head), every MMA tile at full size: w, u
    recompute 2C(K+V); h recompute 4KV; dv_local 2C(K+V); dh recurrence 6KV; dq/dk/dw/dg 6KV + 6CK + 2CV;
    WY backward 10CK + 4CV + 4C^2 -> 16KV + 20CK + 10CV + 4C^2."""
    return 16 * K * V + 20 * C * K + 10 * C * V + 4 * C * C


def bench_backward(args, dev):
    """One step = one kairos_gdn_chunk_bwd call (the whole backward: recompute of the forward's
    intermediates, dv_local, the dh recurrence, dq/dk/dw/dg and the WY backward) at BASELINE config 2,
    or at the Kairos layer's head dims with --model-shape.  Algorithmic bytes: q, k, v, do read and
    dq, dk, dv written once per token-head (7 x 2 B x d), g, beta read and dg, dbeta written, plus h0 and
    dht read and dh0 written per (sequence, head).  --l2norm passes unnormalised q, k with the in-op L2
    norm (the layer's own mode: the op normalises them and its backward goes through the norm)."""
    from kairos_gdn import _lib
    K, V = (256, 512) if args.model_shape else (128, 128)
    B, T, H = 1, args.T, 20
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, 20262, device=dev)
    gen = torch.Generator(device="cpu").manual_seed(20263)
    l2 = 1 if args.l2norm else 0
    if l2:
        q = (q.float() * torch.rand(B, T, H, 1, generator=gen).add_(0.5).to(dev)).to(torch.bfloat16)
        k = (k.float() * torch.rand(B, T, H, 1, generator=gen).add_(0.5).to(dev)).to(torch.bfloat16)
    do = torch.randn(B, T, H, V, generator=gen).to(dev, torch.bfloat16)
    dht = torch.randn(B, H, K, V, generator=gen).to(dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dg = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    db = torch.empty_like(beta)
    dh0 = torch.empty_like(h0)
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_bwd_workspace_size(B, T, H, K, V, 0, _lib.BF16, _lib.BF16, l2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_chunk_bwd", P(q), P(k), P(v), P(g), P(beta), P(h0), P(do), P(dht), P(dq), P(dk), P(dv),
                  P(dg), P(db), P(dh0), None, 0, B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32,
                  K ** -0.5, l2, P(ws), ws_bytes, sp)

    timer = Timer(args)
    res = timer.run(step)
    wall = res["wall_s"]
    med_s = res["step_ms"]["median"] / 1e3
    tok_heads = B * T * H
    # q, k, dq, dk (4 x K) and v, do, dv (3 x V) in bf16; g, dg fp32 and beta, dbeta bf16; h0, dht, dh0 fp32
    alg = tok_heads * (2 * (4 * K + 3 * V) + 12) + B * H * 3 * K * V * 4
    flops = tok_heads * bwd_flops_per_tok_head(K, V)
    print(json.dumps({
        "metric": f"GDN chunk-bwd tokens/s + TFLOP/s at T={T},H={H},dk={K},dv={V}"
                  + (" with use_qk_l2norm_in_kernel=True" if l2 else ""), "value": B * T / wall,
        "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"kairos_gdn_chunk_bwd B={B} T={T} H={H} dk={K} dv={V} chunk 64, bf16 q/k/v/beta/do, "
                               "fp32 g/h0/dht, gradients of q, k, v, g, beta, h0; inputs in HBM",
                   "workspace_bytes": ws_bytes},
        **timer.fields(res),
        "tflops": flops / wall / 1e12, "mfma_peak_frac": flops / wall / 1e12 / PEAK_BF16_TFLOPS,
        "roofline": {"bound": "hbm", "kernel": "whole call (median step)", "achieved": alg / med_s / 1e9,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": alg / med_s / 1e9 / PEAK_HBM_GBS,
                     "alg_bytes": alg, "traffic": None},
    }), flush=True)


# ---------------------------------------------------------------------------
# other rows of the path (each prints its own line)
# ---------------------------------------------------------------------------
def bench_gated_norm(args, dev):
    """The forward with the layer's output norm (kairos_gdn_chunk_fwd_gated_norm): the norm folded into
    the forward (the segment scan's output kernel at config 2; with --model-shape, dk=256 / dv=512, the
    fused K = 256 kernel's loader waves, opt-in there) against the same call with the separate norm
    kernel (KAIROS_GDN_FUSED_NORM=0), A/B in one process; `value` times the library's default form.
    --l2norm passes unnormalised q, k with the in-op L2 norm (the layer's own mode)."""
    from kairos_gdn import _lib
    cfg = CONFIGS[2]
    B, T, H, K, V = cfg["B"], cfg["T"], cfg["H"], cfg["K"], cfg["V"]
    if args.model_shape:
        B, T, H, K, V = 1, args.T, 20, 256, 512
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, cfg["seed"], n_states=B, device=dev)
    l2 = 1 if args.l2norm else 0
    gen = torch.Generator(device="cpu").manual_seed(20263)
    if l2:
        q = (q.float() * torch.rand(B, T, H, 1, generator=gen).add_(0.5).to(dev)).to(torch.bfloat16)
        k = (k.float() * torch.rand(B, T, H, 1, generator=gen).add_(0.5).to(dev)).to(torch.bfloat16)
    gate = torch.randn(B, T, H, V, generator=gen).to(dev, torch.bfloat16)
    w = torch.rand(V, generator=gen).add_(0.5).to(dev)
    lib = _lib.load()
    fold_prev = os.environ.get("KAIROS_GDN_WIDE_NORM_FOLD")
    os.environ["KAIROS_GDN_WIDE_NORM_FOLD"] = "1"        # size the workspace for either form
    ws_bytes = lib.kairos_gdn_chunk_fwd_gated_norm_workspace_size(B, T, H, K, V, 0, _lib.BF16, _lib.BF16, l2)
    if fold_prev is None:
        os.environ.pop("KAIROS_GDN_WIDE_NORM_FOLD")
    else:
        os.environ["KAIROS_GDN_WIDE_NORM_FOLD"] = fold_prev
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    y = torch.empty_like(v)
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_chunk_fwd_gated_norm", P(q), P(k), P(v), P(g), P(beta), None, None, P(h0), P(gate),
                  P(w), None, P(y), P(ht), None, 0, B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16,
                  _lib.F32, _lib.BF16, _lib.F32, K ** -0.5, l2, 1e-5, _lib.ACT_SWISH, P(ws), ws_bytes, sp)

    # at the layer shape "fused" is the norm folded into the fused K = 256 kernel (opt-in there)
    names = ("KAIROS_GDN_FUSED_NORM", "KAIROS_GDN_WIDE_NORM_FOLD")
    prev = {n: os.environ.get(n) for n in names}
    out = {}
    try:
        default = "separate" if args.model_shape else "fused"
        for form, flag in (("separate", "0"), ("fused", "1")):
            if args.default_form_only and form != default:
                continue
            os.environ["KAIROS_GDN_FUSED_NORM"] = flag
            os.environ["KAIROS_GDN_WIDE_NORM_FOLD"] = flag
            timer = Timer(args)
            out[form] = (timer, timer.run(step))
    finally:
        for n, v in prev.items():
            if v is None:
                os.environ.pop(n, None)
            else:
                os.environ[n] = v
    # `value` is the library's default form: folded into seg_out at config 2, the separate norm kernel
    # (by parts beside the pipelined forward) at the layer shape (the fold there is opt-in: measured slower)
    timer, res = out[default]
    med = res["step_ms"]["median"]
    shape = f"T={T},H={H},dk={K},dv={V}" if args.model_shape else "T=32760,H=20,d=128"
    print(json.dumps({
        "metric": f"GDN chunk-fwd + gated RMSNorm (the layer's o_norm) tokens/s at {shape}",
        "value": B * T / (med / 1e3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": res["wall_s"] * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": ("the Kairos layer shape" if args.model_shape else "BASELINE config 2") +
                               f" forward with FusedRMSNormGated({V}, eps=1e-5, swish) on o, bf16 gate, fp32 "
                               "weight, through kairos_gdn_chunk_fwd_gated_norm" +
                               (", use_qk_l2norm_in_kernel=True (unnormalised q, k)" if l2 else ""),
                   "B": B, "T": T, "H": H, "dk": K, "dv": V, "workspace_bytes": ws_bytes},
        **timer.fields(res),
        "default_form": "norm kernel after the forward" if default == "separate" else "norm folded into the forward",
        "forms": {("norm_folded_into_forward" if f == "fused" else "norm_kernel_after_forward"):
                  {"median_ms": r["step_ms"]["median"], "cold_median_ms": (r.get("cold_step_ms") or {}).get("median")}
                  for f, (_, r) in out.items()},
    }), flush=True)


def bench_epilogue(args, dev):
    """Gated RMSNorm (fla FusedRMSNormGated, the layer's o_norm) over config 2's output rows:
    algorithmic bytes = rows * V * (2 + 2 + 2) (read o and the gate, write y, bf16)."""
    from kairos_gdn import _lib
    T, H, V = args.T, 20, 128
    rows = T * H
    gen = torch.Generator(device="cpu").manual_seed(20262)
    x = torch.randn(rows, V, generator=gen).to(dev, torch.bfloat16)
    gate = torch.randn(rows, V, generator=gen).to(dev, torch.bfloat16)
    w = torch.rand(V, generator=gen).add_(0.5).to(dev)
    y = torch.empty_like(x)
    sp = torch.cuda.current_stream(dev).cuda_stream

    def step():
        _lib.call("kairos_gdn_rms_norm_gated", x.data_ptr(), gate.data_ptr(), w.data_ptr(), None, y.data_ptr(),
                  None, _lib.BF16, _lib.BF16, _lib.F32, rows, V, 1e-5, _lib.ACT_SWISH, sp)

    timer = Timer(args)
    res = timer.run(step)
    ms = res["step_ms"]["median"]
    nbytes = rows * V * 6
    gbs = nbytes / (ms / 1e3) / 1e9
    print(json.dumps({
        "metric": "gated RMSNorm epilogue GB/s at T=32760,H=20,dv=128", "value": gbs, "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["wall_s"] * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "FusedRMSNormGated(128, eps=1e-5, swish) on o [T*H, 128] bf16, bf16 gate, "
                               "fp32 weight", "rows": rows},
        **timer.fields(res),
        "roofline": {"bound": "hbm", "kernel": "rmsnorm_gated_kernel", "achieved": gbs, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS, "alg_bytes": nbytes, "traffic": None},
    }), flush=True)


def bench_model_shape(args, dev):
    """The Kairos 4B layer's own head dims (GatedDeltaNet(hidden_size=2560, num_heads=20) with the
    layer defaults head_dim=256, expand_v=2): B=1, H=20, K=256, V=512 at the headline T, bf16.
    FLOPs counted as for the headline metric (every MMA tile at full size)."""
    from kairos_gdn import _lib
    B, T, H, K, V = 1, args.T, 20, 256, 512
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, 20270, device=dev)
    l2 = int(bool(args.l2norm))
    if l2:          # the layer hands the op unnormalised q, k and asks it to normalise them
        q = (q.float() * 3.0).to(torch.bfloat16)
        k = (k.float() * 0.5).to(torch.bfloat16)
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, 0, _lib.BF16, _lib.BF16, l2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_chunk_fwd", P(q), P(k), P(v), P(g), P(beta), None, None, P(h0), P(o), P(ht), None, 0,
                  B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, K ** -0.5, l2, P(ws), ws_bytes,
                  sp)

    timer = Timer(args)
    res = timer.run(step)
    wall = res["wall_s"]
    med_s = res["step_ms"]["median"] / 1e3
    alg = alg_bytes(B * T * H, B * H, K, V)
    tflops = B * T * H * flops_per_tok_head(K, V) / wall / 1e12
    print(json.dumps({
        "metric": "GDN chunk-fwd tokens/s at the Kairos 4B layer shape T=32760,H=20,dk=256,dv=512"
                  + (" with use_qk_l2norm_in_kernel=True" if l2 else ""), "value": T / wall,
        "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"chunk_gated_delta_rule fwd B={B} T={T} H={H} dk={K} dv={V} chunk 64, bf16 "
                               "q/k/v/beta, fp32 g/h0, output_final_state, inputs in HBM"
                               + (", use_qk_l2norm_in_kernel=True (unnormalised q, k)" if l2 else ""),
                   "workspace_bytes": ws_bytes},
        **timer.fields(res),
        "tflops": tflops, "mfma_peak_frac": tflops / PEAK_BF16_TFLOPS,
        "hbm_gbs_whole_op": alg / wall / 1e9,
        "roofline": {"bound": "hbm", "kernel": "whole call (median step)", "achieved": alg / med_s / 1e9,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": alg / med_s / 1e9 / PEAK_HBM_GBS,
                     "alg_bytes": alg,
                     "traffic": measured_call_traffic(MODEL_L2_TRAFFIC_FILE, "chunk_fwd_model_shape_l2norm") if l2
                     else measured_call_traffic(MODEL_TRAFFIC_FILE, "chunk_fwd_model_shape")},
    }), flush=True)


def bench_recurrent(args, dev):
    """Decoding step of the layer's short-sequence mode (fused_recurrent_gated_delta_rule, q_len <= 64):
    B=8 streams, one token each, at the Kairos 4B layer's head dims (H=20, K=256, V=512), bf16 q/k/v,
    fp32 state carried in and out.  Algorithmic bytes = state read + write (2 * B*H*K*V*4) + the
    token's q, k, v, o, g, beta; the kernel is bound by the two state passes in HBM."""
    from kairos_gdn import _lib
    B, T, H, K, V = 8, 1, 20, 256, 512
    q, k, v, g, beta, _ = make_inputs(B, T, H, K, V, 20271, device=dev)
    h0 = (0.02 * torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(1))).to(dev)
    o = torch.empty_like(v)
    ht = torch.empty_like(h0)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_fused_recurrent_fwd", P(q), P(k), P(v), P(g), None, None, P(beta), P(h0), P(o), P(ht),
                  None, 0, B, T, H, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.F32, _lib.F32, _lib.BF16, 1, _lib.F32,
                  K ** -0.5, 1, sp)

    timer = Timer(args)
    res = timer.run(step)
    ms = res["step_ms"]["median"]
    nbytes = 2 * B * H * K * V * 4 + B * T * H * (2 * K * 2 + 2 * V * 2 + 4 + 2)
    gbs = nbytes / (ms / 1e3) / 1e9
    print(json.dumps({
        "metric": "GDN fused_recurrent decode step (B=8, T=1, H=20, dk=256, dv=512) GB/s", "value": gbs,
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["wall_s"] * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "fused_recurrent_gated_delta_rule fwd, 8 streams x 1 token, H=20 dk=256 dv=512, "
                               "bf16 q/k/v/beta, fp32 g and state, in-kernel q/k L2 norm, state in HBM"},
        **timer.fields(res),
        "roofline": {"bound": "hbm", "kernel": "fused_recurrent_kernel", "achieved": gbs, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS, "alg_bytes": nbytes, "traffic": None},
    }), flush=True)


def bench_prologue(args, dev):
    """The layer's prologue at the Kairos 4B shape (hidden 2560 -> H=20, dk=256, dv=512): causal conv
    k=4 + SiLU over the q and k projections (D=5120, fused per-head L2 norm) and the v projection
    (D=10240), bf16, caches out, plus the gates.  Algorithmic bytes = each projection read once and
    written once (2 + 2 B per element) + caches + gate rows."""
    from kairos_gdn import _lib
    T, H, K, V, W = args.T, 20, 256, 512, 4
    gen = torch.Generator(device="cpu").manual_seed(20272)
    xs = [torch.randn(T, D, generator=gen).to(dev, torch.bfloat16) for D in (H * K, H * K, H * V)]
    ws = [(0.5 * torch.randn(x.shape[1], W, generator=gen)).to(dev, torch.bfloat16) for x in xs]
    ys = [torch.empty_like(x) for x in xs]
    hs = [torch.empty(1, x.shape[1], W, dtype=torch.bfloat16, device=dev) for x in xs]
    a = torch.randn(T, H, generator=gen).to(dev, torch.bfloat16)
    b = torch.randn(T, H, generator=gen).to(dev, torch.bfloat16)
    A_log = torch.rand(H, generator=gen).mul_(16).log_().to(dev)
    dt_bias = torch.randn(H, generator=gen).to(dev)
    g = torch.empty(T, H, dtype=torch.float32, device=dev)
    beta = torch.empty_like(b)
    sp = torch.cuda.current_stream(dev).cuda_stream
    l2 = (K, K, 0)
    P = lambda t: t.data_ptr()  # noqa: E731

    def step():
        for x, w, y, h, hd in zip(xs, ws, ys, hs, l2):
            _lib.call("kairos_gdn_causal_conv1d_fwd", P(x), P(w), None, None, P(y), P(h), None, 0, 1, T, x.shape[1], W,
                      _lib.BF16, _lib.BF16, 1, hd, sp)
        _lib.call("kairos_gdn_gates_fwd", P(a), P(b), P(A_log), P(dt_bias), P(g), P(beta), T, H, _lib.BF16, _lib.BF16,
                  _lib.F32, 0, sp)

    timer = Timer(args)
    res = timer.run(step)
    ms = res["step_ms"]["median"]
    nbytes = sum(x.numel() * 4 + x.shape[1] * W * 2 * 2 for x in xs) + T * H * (2 + 2 + 4 + 2)
    gbs = nbytes / (ms / 1e3) / 1e9
    print(json.dumps({
        "metric": "GDN layer prologue (conv k=4 + SiLU on q/k/v with fused q/k L2 norm, gates) GB/s at "
                  "T=32760, H=20, dk=256, dv=512", "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": res["wall_s"] * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "kairos_gdn_causal_conv1d_fwd x3 (q, k: D=5120 with per-head L2 norm; v: D=10240), "
                               "bf16, W=4, caches out, + kairos_gdn_gates_fwd (T x 20)"},
        **timer.fields(res),
        "roofline": {"bound": "hbm", "kernel": "conv1d_kernel", "achieved": gbs, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS, "alg_bytes": nbytes, "traffic": None},
    }), flush=True)


def bench_prologue_fused(args, dev):
    """The layer's prologue folded into the forward (kairos_gdn_chunk_fwd_conv) against the same work
    as two steps (kairos_gdn_causal_conv1d_fwd on q, k with the per-head L2 norm and on v, then
    kairos_gdn_chunk_fwd), one process, same inputs: the Kairos 4B layer's shape (T=32760, H=20,
    dk=256, dv=512), bf16 projections, conv caches in and out, h0 and final state.  The value is the
    fused call's tokens/s; algorithmic bytes = the projections, gates and output once, the states
    and caches (the convolved q, k, v are not counted: the fused call need not store them)."""
    from kairos_gdn import _lib
    B, T, H, K, V, W = 1, args.T, 20, 256, 512, 4
    gen = torch.Generator(device="cpu").manual_seed(20274)
    DK, DV = H * K, H * V
    xs = [torch.randn(B * T, D, generator=gen).to(dev, torch.bfloat16) for D in (DK, DK, DV)]
    ws = [(0.5 * torch.randn(x.shape[1], W, generator=gen)).to(dev, torch.bfloat16) for x in xs]
    cin = [torch.randn(B, x.shape[1], W, generator=gen).to(dev, torch.bfloat16) for x in xs]
    cout = [torch.empty_like(c) for c in cin]
    ys = [torch.empty_like(x) for x in xs]
    g = (-torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen))).to(dev)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).to(dev, torch.bfloat16)
    h0 = (0.02 * torch.randn(B, H, K, V, generator=gen)).to(dev)
    o = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    lib = _lib.load()
    ws_f = lib.kairos_gdn_chunk_fwd_conv_workspace_size(B, T, H, K, V, 0, 1)
    ws_s = lib.kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, 0, _lib.BF16, _lib.BF16, 0)
    wsf = torch.empty(max(ws_f, 1), dtype=torch.uint8, device=dev)
    wss = torch.empty(max(ws_s, 1), dtype=torch.uint8, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def fused():
        _lib.call("kairos_gdn_chunk_fwd_conv", *(P(x) for x in xs), *(P(w) for w in ws), None, None, None,
                  *(P(c) for c in cin), *(P(c) for c in cout), _lib.BF16, P(g), P(beta), P(h0), P(o), P(ht), None, 0,
                  B, T, H, K, V, _lib.F32, _lib.BF16, _lib.F32, K ** -0.5, 1, P(wsf), ws_f, sp)

    def two_step():
        for x, w, y, c0, c1, hd in zip(xs, ws, ys, cin, cout, (K, K, 0)):
            _lib.call("kairos_gdn_causal_conv1d_fwd", P(x), P(w), None, P(c0), P(y), P(c1), None, 0, B, T, x.shape[1],
                      W, _lib.BF16, _lib.BF16, 1, hd, sp)
        _lib.call("kairos_gdn_chunk_fwd", P(ys[0]), P(ys[1]), P(ys[2]), P(g), P(beta), None, None, P(h0), P(o), P(ht),
                  None, 0, B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, K ** -0.5, 0, P(wss),
                  ws_s, sp)

    timer = Timer(args)
    res = timer.run(fused)
    res2 = Timer(args).run(two_step)
    wall = res["wall_s"]
    med_s = res["step_ms"]["median"] / 1e3
    alg = B * T * (2 * DK + DV) * 2 + B * T * H * (4 + 2) + B * T * H * V * 2 + 2 * B * H * K * V * 4 \
        + 2 * sum(c.numel() * 2 for c in cin)
    print(json.dumps({
        "metric": "GDN layer prologue + chunk-fwd in one call, tokens/s at T=32760,H=20,dk=256,dv=512",
        "value": T / wall, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": wall * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"kairos_gdn_chunk_fwd_conv B={B} T={T} H={H} dk={K} dv={V}: conv k=4 + SiLU on "
                               "the q/k/v projections, in-op L2 norm, conv caches in/out, h0, final state; "
                               "against kairos_gdn_causal_conv1d_fwd x3 + kairos_gdn_chunk_fwd",
                   "workspace_bytes": ws_f},
        **timer.fields(res),
        "two_step_ms": {"median": res2["step_ms"]["median"], "wall": res2["wall_s"] * 1e3,
                        "cold_median": res2.get("cold_step_ms", {}).get("median")},
        "speedup_vs_two_step": res2["step_ms"]["median"] / res["step_ms"]["median"],
        "roofline": {"bound": "hbm", "kernel": "whole call (median step)", "achieved": alg / med_s / 1e9,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": alg / med_s / 1e9 / PEAK_HBM_GBS, "alg_bytes": alg,
                     "traffic": None},
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--warmup-seconds", type=float, default=1.5,
                    help="minimum wall time of the untimed warm-up (clocks reach steady state)")
    ap.add_argument("--no-cold", action="store_true", help="skip the cold-cache (flushed) steps")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4],
                    help="BASELINE config to measure (2 = the headline; 4 = the 21-frame fp8 streaming rollout)")
    ap.add_argument("--l2norm", action="store_true",
                    help="run the op with use_qk_l2norm_in_kernel=True on unnormalised q, k (configs 1-3 and "
                         "--model-shape)")
    ap.add_argument("--T", type=int, default=32760)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run only a plain elementwise copy of MIB MiB (fp32 y = x * 1) 5 times and exit: the "
                         "reference kernel of known traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--epilogue", action="store_true",
                    help="measure only the gated RMSNorm epilogue (kairos_gdn_rms_norm_gated) on o-shaped rows")
    ap.add_argument("--gated-norm", action="store_true",
                    help="measure the forward with the layer's gated RMSNorm (folded into the forward against "
                         "the separate norm kernel); config 2, or the layer shape with --model-shape")
    ap.add_argument("--default-form-only", action="store_true",
                    help="with --gated-norm: time only the library's default form (for a profile of it alone)")
    ap.add_argument("--model-shape", action="store_true",
                    help="measure the Kairos 4B layer's head dims (dk=256, dv=512, H=20) at --T")
    ap.add_argument("--recurrent", action="store_true",
                    help="measure the short-sequence mode's decoding step (8 streams x 1 token at dk=256, dv=512)")
    ap.add_argument("--backward", action="store_true",
                    help="measure the backward pass (kairos_gdn_chunk_bwd) at config 2's shape (--model-shape: the "
                         "Kairos layer's dk=256, dv=512); prints its own JSON line")
    ap.add_argument("--prologue-fused", action="store_true",
                    help="the layer's prologue folded into the forward (kairos_gdn_chunk_fwd_conv) against the "
                         "two-step conv + forward, at the Kairos 4B layer shape")
    ap.add_argument("--prologue", action="store_true",
                    help="measure the layer prologue (causal conv + SiLU + q/k L2 norm, gates) at the model shape")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build runs the op on a single GPU and has no multi-GPU "
              f"path (got --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)

    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        x = torch.ones(n, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        for _ in range(5):
            torch.mul(x, 1.0, out=y)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": 4 * n, "calibrate_copy_bytes_written": 4 * n}), flush=True)
        return

    import kairos_gdn  # noqa: F401
    if args.backward:
        bench_backward(args, dev)
    elif args.epilogue:
        bench_epilogue(args, dev)
    elif args.gated_norm:
        bench_gated_norm(args, dev)
    elif args.model_shape:
        bench_model_shape(args, dev)
    elif args.recurrent:
        bench_recurrent(args, dev)
    elif args.prologue_fused:
        bench_prologue_fused(args, dev)
    elif args.prologue:
        bench_prologue(args, dev)
    elif args.config == 4:
        bench_streaming(args, dev)
    else:
        bench_chunk(args, dev, args.config)


if __name__ == "__main__":
    main()
