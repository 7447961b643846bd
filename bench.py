"""Benchmark of the MI355X chunked GatedDeltaNet forward (BASELINE.json metric).

One step = one chunk_gated_delta_rule forward over BASELINE config 2
(B=1, T=32760, H=20, dk=dv=128, chunk 64, bf16 q/k/v/beta, fp32 g and h0,
output_final_state=True) with inputs resident in HBM, through the C ABI
(kairos_gdn_chunk_fwd).  Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu-baseline]
  python bench.py --calibrate-copy 1024     # reference copy kernel for rocprofv3 counter scaling
  python bench.py --epilogue                # the gated RMSNorm output epilogue on config 2's o
  python bench.py --model-shape             # the Kairos 4B layer's head dims dk=256, dv=512
  python bench.py --recurrent               # the short-sequence mode's decoding step (fused_recurrent)
  python bench.py --prologue                # the layer prologue: causal conv + SiLU (+ q/k L2 norm), gates

`value` is tokens/s of whole forward calls (wall clock between two device
synchronisations around `steps` back-to-back calls).  Per-kernel times come
from a second loop in which the library records hipEvents on the launch
stream around each of its kernels (kairos_gdn_profile_begin/_end).  The
roofline block is the dominant kernel's algorithmic HBM bytes per launch over
its average duration; `traffic` is that kernel's measured HBM bytes per launch
from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary, when present.
"""
import argparse
import ctypes
import json
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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "chunk_fwd_config2_hbm_traffic.md")


def flops_per_tok_head(K, V):
    """Algorithmic FLOPs per (token, head), every MMA tile counted at full size."""
    return 6 * K * V + 6 * C * K + 4 * C * V


def kernel_models(B, T, H, K, V, L, s=2, s_g=4, s_b=2):
    """Algorithmic HBM bytes (compulsory reads + writes) and FLOPs of one launch of each kernel.

    seg_prep reads k, g, beta and writes one chunk record per (chunk, head):
    the bf16 inverse Ai (64 x 64) and eight fp32 vectors of 64 (cumulative
    gates and the gate / beta products the later kernels use), RECORD bytes.
    seg_out reads q, k, v, the records and the segment initial states, writes
    o and final_state; seg_trans reads k, v and the records of every segment
    but the last of each sequence and writes its [M | R]; seg_combine reads
    [M | R] and h0 and writes the segment initial states.  FLOPs count every
    MMA tile at full size: K.K^T (2CK per token) in seg_prep, the rest of the
    chunk algebra in seg_out, w, u and the two [M | R] products in seg_trans.
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


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 summary, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for ln in f:
                m = re.match(r"\s*traffic_bytes_per_launch\s+(\S+)\s+(\d+)", ln)
                if m and m.group(1) == kernel:
                    return int(m.group(2))
    except OSError:
        pass
    return None


def make_inputs(B, T, H, K, V, seed, device):
    g_ = torch.Generator(device="cpu").manual_seed(seed)

    def unit(shape):
        x = torch.randn(shape, generator=g_)
        return torch.nn.functional.normalize(x, dim=-1)
    q = unit((B, T, H, K)).to(device, torch.bfloat16)
    k = unit((B, T, H, K)).to(device, torch.bfloat16)
    v = torch.randn((B, T, H, V), generator=g_).to(device, torch.bfloat16)
    beta = torch.sigmoid(torch.randn((B, T, H), generator=g_)).to(device, torch.bfloat16)
    g = (-torch.nn.functional.softplus(torch.randn((B, T, H), generator=g_))).to(device, torch.float32)
    h0 = (0.02 * torch.randn((B, H, K, V), generator=g_)).to(device, torch.float32)
    return q, k, v, g, beta, h0


def cpu_baseline(T, H, K, V, seed, min_seconds=10.0):
    """Time the numpy oracle (bf16-emulating chunked restatement) on the host cores.

    The sample is the full config (all H heads of T tokens), repeated until at
    least `min_seconds` of CPU work; the rate is the median over repeats.
    """
    sys.path.insert(0, ROOT)
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits
    from oracle import gdn_oracle as O
    cores = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(seed)

    def unit(shape):
        x = rng.standard_normal(shape, dtype=np.float32)
        return O.to_bf16(x / np.sqrt((x * x).sum(-1, keepdims=True)))
    q, k = unit((1, T, H, K)), unit((1, T, H, K))
    v = O.to_bf16(rng.standard_normal((1, T, H, V), dtype=np.float32))
    beta = O.to_bf16(1 / (1 + np.exp(-rng.standard_normal((1, T, H), dtype=np.float32))))
    g = (-np.logaddexp(0, rng.standard_normal((1, T, H), dtype=np.float32))).astype(np.float32)
    h0 = (0.02 * rng.standard_normal((1, H, K, V), dtype=np.float32)).astype(np.float32)
    times = []
    with threadpool_limits(cores):
        t_start = time.perf_counter()
        while not times or (time.perf_counter() - t_start < min_seconds and len(times) < 10):
            t0 = time.perf_counter()
            O.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True, dtype="bf16")
            times.append(time.perf_counter() - t0)
        blas = [i.get("num_threads") for i in threadpool_info()]
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    dt = statistics.median(times)
    return {"value": T / dt, "unit": "tokens/s", "cores": max(blas) if blas else cores, "kind": "port",
            "sample": f"numpy oracle (oracle/gdn_oracle.py, bf16 cast points) on the full workload "
                      f"(T={T}, all {H} heads), {len(times)} runs in {sum(times):.1f} s, median {dt:.2f} s per "
                      f"forward; host CPU: {model}"}


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

    for _ in range(args.warmup):
        step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = rows * V * 6
    gbs = nbytes / (ms / 1e3) / 1e9
    print(json.dumps({
        "metric": "gated RMSNorm epilogue GB/s at T=32760,H=20,dv=128", "value": gbs, "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "FusedRMSNormGated(128, eps=1e-5, swish) on o [T*H, 128] bf16, bf16 gate, "
                               "fp32 weight", "rows": rows},
        "roofline": {"bound": "hbm", "kernel": "rmsnorm_gated_kernel", "achieved": gbs, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS, "traffic": None},
    }), flush=True)


def bench_model_shape(args, dev):
    """The Kairos 4B layer's own head dims (GatedDeltaNet(hidden_size=2560, num_heads=20) with the
    layer defaults head_dim=256, expand_v=2): B=1, H=20, K=256, V=512 at the headline T, bf16.
    These dims run the stage kernels (prepare -> fwd_h -> fwd_o) with the reference's
    intermediates; FLOPs counted as for the headline metric (every MMA tile at full size)."""
    from kairos_gdn import _lib
    B, T, H, K, V = 1, args.T, 20, 256, 512
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, 20270, dev)
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, 0, _lib.BF16, _lib.BF16, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_chunk_fwd", P(q), P(k), P(v), P(g), P(beta), None, None, P(h0), P(o), P(ht), None, 0,
                  B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, K ** -0.5, 0, P(ws), ws_bytes,
                  sp)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    tflops = B * T * H * flops_per_tok_head(K, V) / wall / 1e12
    nbytes = B * T * H * (2 * K * 2 + 2 * V * 2 + 4 + 2) + 2 * B * H * K * V * 4
    print(json.dumps({
        "metric": "GDN chunk-fwd tokens/s at the Kairos 4B layer shape T=32760,H=20,dk=256,dv=512", "value": T / wall,
        "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"chunk_gated_delta_rule fwd B={B} T={T} H={H} dk={K} dv={V} chunk 64, bf16 "
                               "q/k/v/beta, fp32 g/h0, output_final_state, inputs in HBM (stage kernels)"},
        "tflops": tflops, "mfma_peak_frac": tflops / PEAK_BF16_TFLOPS,
        "hbm_gbs_whole_op": nbytes / wall / 1e9,
    }), flush=True)


def bench_recurrent(args, dev):
    """Decoding step of the layer's short-sequence mode (fused_recurrent_gated_delta_rule, q_len <= 64):
    B=8 streams, one token each, at the Kairos 4B layer's head dims (H=20, K=256, V=512), bf16 q/k/v,
    fp32 state carried in and out.  Algorithmic bytes = state read + write (2 * B*H*K*V*4) + the
    token's q, k, v, o, g, beta; the kernel is bound by the two state passes in HBM."""
    from kairos_gdn import _lib
    B, T, H, K, V = 8, 1, 20, 256, 512
    q, k, v, g, beta, _ = make_inputs(B, T, H, K, V, 20271, dev)
    h0 = (0.02 * torch.randn(B, H, K, V, generator=torch.Generator().manual_seed(1))).to(dev)
    o = torch.empty_like(v)
    ht = torch.empty_like(h0)
    sp = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_fused_recurrent_fwd", P(q), P(k), P(v), P(g), None, None, P(beta), P(h0), P(o), P(ht),
                  None, 0, B, T, H, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.F32, _lib.F32, _lib.BF16, 1, _lib.F32,
                  K ** -0.5, 1, sp)

    for _ in range(args.warmup):
        step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = 2 * B * H * K * V * 4 + B * T * H * (2 * K * 2 + 2 * V * 2 + 4 + 2)
    gbs = nbytes / (ms / 1e3) / 1e9
    print(json.dumps({
        "metric": "GDN fused_recurrent decode step (B=8, T=1, H=20, dk=256, dv=512) GB/s", "value": gbs,
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "fused_recurrent_gated_delta_rule fwd, 8 streams x 1 token, H=20 dk=256 dv=512, "
                               "bf16 q/k/v/beta, fp32 g and state, in-kernel q/k L2 norm, state in HBM"},
        "roofline": {"bound": "hbm", "kernel": "fused_recurrent_kernel", "achieved": gbs, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS, "traffic": None},
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

    for _ in range(args.warmup):
        step()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = sum(x.numel() * 4 + x.shape[1] * W * 2 * 2 for x in xs) + T * H * (2 + 2 + 4 + 2)
    gbs = nbytes / (ms / 1e3) / 1e9
    print(json.dumps({
        "metric": "GDN layer prologue (conv k=4 + SiLU on q/k/v with fused q/k L2 norm, gates) GB/s at "
                  "T=32760, H=20, dk=256, dv=512", "value": gbs, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "kairos_gdn_causal_conv1d_fwd x3 (q, k: D=5120 with per-head L2 norm; v: D=10240), "
                               "bf16, W=4, caches out, + kairos_gdn_gates_fwd (T x 20)"},
        "roofline": {"bound": "hbm", "kernel": "conv1d_kernel", "achieved": gbs, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS, "traffic": None},
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--T", type=int, default=32760)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run only a plain elementwise copy of MIB MiB (fp32 y = x * 1) 5 times and exit: the "
                         "reference kernel of known traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--epilogue", action="store_true",
                    help="measure only the gated RMSNorm epilogue (kairos_gdn_rms_norm_gated) on o-shaped rows "
                         "[T*H, V] bf16 with a bf16 gate and fp32 weight; prints its own JSON line")
    ap.add_argument("--model-shape", action="store_true",
                    help="measure the Kairos 4B layer's head dims (dk=256, dv=512, H=20) at --T; prints its own "
                         "JSON line")
    ap.add_argument("--recurrent", action="store_true",
                    help="measure the short-sequence mode's decoding step (kairos_gdn_fused_recurrent_fwd, 8 streams "
                         "x 1 token at dk=256, dv=512); prints its own JSON line")
    ap.add_argument("--prologue", action="store_true",
                    help="measure the layer prologue (causal conv + SiLU + q/k L2 norm, gates) at the model shape; "
                         "prints its own JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
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
    from kairos_gdn import _lib
    if args.epilogue:
        bench_epilogue(args, dev)
        return
    if args.model_shape:
        bench_model_shape(args, dev)
        return
    if args.recurrent:
        bench_recurrent(args, dev)
        return
    if args.prologue:
        bench_prologue(args, dev)
        return
    B, T, H, K, V = 1, args.T, 20, 128, 128
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, 20262, dev)
    scale = K ** -0.5
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, 0, _lib.BF16, _lib.BF16, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    o = torch.empty_like(v)
    ht = torch.empty(B, H, K, V, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def step():
        _lib.call("kairos_gdn_chunk_fwd", P(q), P(k), P(v), P(g), P(beta), None, None, P(h0), P(o), P(ht), None, 0,
                  B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, scale, 0, P(ws), ws_bytes, sp)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps

    # ---- per-kernel times: hipEvents recorded by the library on the launch stream
    lib.kairos_gdn_profile_begin()
    for _ in range(args.steps):
        step()
    avg = (ctypes.c_double * len(KERNELS))()
    ncalls = lib.kairos_gdn_profile_end(avg, len(KERNELS))
    if ncalls != args.steps:
        raise RuntimeError(f"kernel timing recorded {ncalls} calls: {lib.kairos_gdn_last_error().decode()}")
    per = {n: avg[i] for i, n in enumerate(KERNELS)}

    L = lib.kairos_gdn_segment_chunks(B, T, H, 0)
    models = kernel_models(B, T, H, K, V, L)
    dom = max(KERNELS, key=lambda n: per[n])
    dom_s = per[dom] / 1e3
    achieved = models[dom]["bytes"] / dom_s / 1e9
    traffic = measured_traffic(dom)
    tok = B * T
    flops = B * T * H * flops_per_tok_head(K, V)
    tflops = flops / wall / 1e12
    nc = (T + C - 1) // C
    out = {
        "metric": METRIC,
        "value": tok / wall,
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
        "config": {"workload": f"BASELINE config 2: chunk_gated_delta_rule fwd B={B} T={T} H={H} dk=dv={K} "
                               "chunk 64, bf16 q/k/v/beta, fp32 g/h0, output_final_state, inputs in HBM",
                   "segments_per_sequence": (nc + L - 1) // L, "chunks_per_segment": L},
        "tflops": tflops,
        "mfma_peak_frac": tflops / PEAK_BF16_TFLOPS,
        "hbm_gbs_whole_op": (B * T * H * (2 * K * 2 + 2 * V * 2 + 4 + 2) + 2 * B * H * K * V * 4) / wall / 1e9,
        "kernels_ms": per,
        "kernels_tflops": {n: models[n]["flops"] / (per[n] / 1e3) / 1e12 if per[n] > 0 else 0.0 for n in KERNELS},
        "kernels_gbs": {n: models[n]["bytes"] / (per[n] / 1e3) / 1e9 if per[n] > 0 else 0.0 for n in KERNELS},
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": traffic,
        },
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(T, H, K, V, 20262)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
