"""Benchmark of the MI355X chunked GatedDeltaNet forward (BASELINE.json metric).

One step = one chunk_gated_delta_rule forward over BASELINE config 2
(B=1, T=32760, H=20, dk=dv=128, chunk 64, bf16 q/k/v/beta, fp32 g and h0,
output_final_state=True) with inputs resident in HBM.  Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]

Per-kernel times come from HIP events recorded on the launch stream around
each stage (prepare, fwd_h, fwd_o) in a separate staged loop; the roofline
block uses the slowest kernel's algorithmic bytes per launch.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kairos-sensenova_amd"))

import torch  # noqa: E402

METRIC = "GDN chunk-fwd tokens/s + TFLOP/s (% bf16 MFMA peak) at T=32760,H=20,d=128"
PEAK_BF16_TFLOPS = 2516.6      # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
C = 64


def flops_per_tok_head(K, V):
    """Algorithmic FLOPs per (token, head), every MMA tile counted at full size."""
    return 6 * K * V + 6 * C * K + 4 * C * V


def kernel_models(B, T, H, K, V, s=2):
    """Per-launch algorithmic FLOPs and HBM bytes of each kernel (compulsory reads + writes)."""
    tok = B * T * H
    nch = B * ((T + C - 1) // C) * H
    return {
        # reads k, v, g, beta; writes w, u, gc
        "prepare": dict(flops=tok * 2 * C * (2 * K + V),
                        bytes=tok * (K * s + V * s + 4 + s) + tok * (K * s + V * s + 4)),
        # reads k, w, u, gc, h0; writes state snapshots, v_new, final state
        "fwd_h": dict(flops=tok * 4 * K * V,
                      bytes=tok * (K * s + K * s + V * s + 4) + nch * K * V * s + tok * V * s + 2 * B * H * K * V * 4),
        # reads q, k, snapshots, v_new, gc; writes o
        "fwd_o": dict(flops=tok * (2 * K * V + 2 * C * (K + V)),
                      bytes=tok * (K * s * 2 + V * s + 4) + nch * K * V * s + tok * V * s),
    }


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


def cpu_baseline(T, H, K, V, heads, seed):
    """Time the numpy oracle (bf16-emulating chunked restatement) on `heads` of the config on the host."""
    sys.path.insert(0, ROOT)
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits
    from oracle import gdn_oracle as O
    cores = min(os.cpu_count() or 1, 16)
    rng = np.random.default_rng(seed)
    def unit(shape):
        x = rng.standard_normal(shape, dtype=np.float32)
        return O.to_bf16(x / np.sqrt((x * x).sum(-1, keepdims=True)))
    q, k = unit((1, T, heads, K)), unit((1, T, heads, K))
    v = O.to_bf16(rng.standard_normal((1, T, heads, V), dtype=np.float32))
    beta = O.to_bf16(1 / (1 + np.exp(-rng.standard_normal((1, T, heads), dtype=np.float32))))
    g = (-np.logaddexp(0, rng.standard_normal((1, T, heads), dtype=np.float32))).astype(np.float32)
    h0 = (0.02 * rng.standard_normal((1, heads, K, V), dtype=np.float32)).astype(np.float32)
    with threadpool_limits(cores):
        t0 = time.perf_counter()
        O.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True, dtype="bf16")
        dt = time.perf_counter() - t0
        blas = [i.get("num_threads") for i in threadpool_info()]
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    # tokens/s of the full H-head config: the sample covers heads/H of the work
    value = T * heads / H / dt
    return {"value": value, "unit": "tokens/s", "cores": max(blas) if blas else cores, "kind": "port",
            "sample": f"numpy oracle (oracle/gdn_oracle.py, bf16 cast points) on T={T}, {heads} of {H} heads; "
                      f"{dt:.2f} s; rate scaled to all {H} heads; host CPU: {model}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=2)
    ap.add_argument("--T", type=int, default=32760)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run only a plain elementwise copy of MIB MiB (fp32 y = x * 1) 5 times and exit: the "
                         "reference kernel of known traffic that scales rocprofv3 FETCH_SIZE / WRITE_SIZE")
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

    import kairos_gdn
    from kairos_gdn import _lib
    B, T, H, K, V = 1, args.T, 20, 128, 128
    q, k, v, g, beta, h0 = make_inputs(B, T, H, K, V, 20262, dev)
    scale = K ** -0.5
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_fwd_workspace_size(B, T, H, K, V, 0, _lib.BF16, _lib.BF16, 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
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

    # ---- per-kernel times: the same three launches issued stage by stage, HIP events on the launch stream
    nc = lib.kairos_gdn_num_chunks_bound(B, T, 0)
    gc = torch.empty(B, T, H, dtype=torch.float32, device=dev)
    w = torch.empty(B, T, H, K, dtype=torch.bfloat16, device=dev)
    uT = torch.empty(nc, H, V, C, dtype=torch.bfloat16, device=dev)
    hT = torch.empty(nc, H, V, K, dtype=torch.bfloat16, device=dev)
    vnT = torch.empty(nc, H, V, C, dtype=torch.bfloat16, device=dev)
    names = ["prepare", "fwd_h", "fwd_o"]

    def stages(ev=None):
        if ev: ev[0].record(stream)
        _lib.call("kairos_gdn_prepare_wy", P(k), P(v), P(g), P(beta), None, P(gc), P(w), P(uT), None, None, None, 0,
                  B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, None, 0, sp)
        if ev: ev[1].record(stream)
        _lib.call("kairos_gdn_fwd_h", P(k), None, P(w), P(uT), P(gc), P(h0), P(hT), P(vnT), P(ht), None, 0,
                  B, T, H, K, V, _lib.BF16, _lib.BF16, _lib.F32, None, 0, sp)
        if ev: ev[2].record(stream)
        _lib.call("kairos_gdn_fwd_o", P(q), P(k), None, None, P(hT), P(vnT), P(gc), P(o), scale, None, 0,
                  B, T, H, K, V, _lib.BF16, _lib.BF16, None, 0, sp)
        if ev: ev[3].record(stream)

    for _ in range(max(2, args.warmup)):
        stages()
    per = {n: 0.0 for n in names}
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    for i in range(args.steps):
        stages(evs[i])
    torch.cuda.synchronize()
    for i in range(args.steps):
        for j, n in enumerate(names):
            per[n] += evs[i][j].elapsed_time(evs[i][j + 1]) / args.steps    # ms

    tok = B * T
    flops = B * T * H * flops_per_tok_head(K, V)
    models = kernel_models(B, T, H, K, V)
    dom = max(names, key=lambda n: per[n])
    dom_s = per[dom] / 1e3
    achieved = models[dom]["bytes"] / dom_s / 1e9
    tflops = flops / wall / 1e12
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
                               "chunk 64, bf16 q/k/v/beta, fp32 g/h0, output_final_state, inputs in HBM"},
        "tflops": tflops,
        "mfma_peak_frac": tflops / PEAK_BF16_TFLOPS,
        "kernels_ms": per,
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_GBS,
            "traffic": None,
        },
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(T, H, K, V, args.cpu_heads, 20262)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
