"""Parity at full size on every head: the oracle over groups of heads in child processes.

At the Kairos layer's shape (T = 32760, H = 20, K = 256, V = 512) the numpy
oracle needs about 4 s per head, so a single process would spend minutes on
one comparison.  Heads are independent, so the inputs and the HIP path's
outputs are written once to a scratch directory (bf16 tensors as their 16-bit
patterns, read back exactly) and child processes, started fresh ("spawn"; they
import only numpy and the oracle), run the oracle on a few heads each and
return sums of squares; the parent combines them into the relative L2 error of
fla's get_err_ratio over all heads.  This module is test infrastructure and
imports no torch.
"""
from __future__ import annotations

import math
import multiprocessing as mp
import os
import shutil
import tempfile
from concurrent.futures import ProcessPoolExecutor, as_completed

import numpy as np


_THREAD_VARS = ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS")


def _to_bits(x: np.ndarray) -> np.ndarray:
    """bf16-valued float32 array -> its 16-bit patterns (exact)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    assert not np.any(u & 0xFFFF), "array holds values that are not bf16"
    return (u >> 16).astype(np.uint16)


def _from_bits(u: np.ndarray) -> np.ndarray:
    return (np.asarray(u).astype(np.uint32) << 16).view(np.float32)


class Scratch:
    """A directory of .npy files shared with the child processes; removed on exit."""

    def __init__(self):
        self.path = tempfile.mkdtemp(prefix="kgdn_oracle_")

    def put(self, name: str, x, bf16: bool = False):
        if x is None:
            return
        np.save(os.path.join(self.path, name + ".npy"), _to_bits(x) if bf16 else np.ascontiguousarray(x))
        with open(os.path.join(self.path, name + ".kind"), "w") as f:
            f.write("bf16" if bf16 else "raw")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        shutil.rmtree(self.path, ignore_errors=True)


def _load(d: str, name: str, heads, axis: int):
    p = os.path.join(d, name + ".npy")
    if not os.path.exists(p):
        return None
    a = np.load(p, mmap_mode="r")
    idx = [slice(None)] * a.ndim
    idx[axis] = heads
    a = np.asarray(a[tuple(idx)])
    with open(os.path.join(d, name + ".kind")) as f:
        return _from_bits(a) if f.read() == "bf16" else a.astype(np.float32)


def _sums(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.sum(np.square(got - ref))), float(np.sum(np.square(ref))), ref.size


def _fwd_job(args):
    d, heads, kw = args
    from oracle import gdn_oracle as O
    x = {n: _load(d, n, heads, 2) for n in ("q", "k", "v", "g", "beta")}
    h0 = _load(d, "h0", heads, 1)
    o_r, ht_r = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=h0,
                                         output_final_state=True, **kw)
    out = {"o": _sums(_load(d, "o", heads, 2), o_r)}
    ht = _load(d, "ht", heads, 1)
    if ht is not None:
        out["ht"] = _sums(ht, ht_r)
    return out


def _bwd_job(args):
    d, heads, kw = args
    from oracle import gdn_oracle_bwd as OB
    x = {n: _load(d, n, heads, 2) for n in ("q", "k", "v", "g", "beta", "do")}
    h0 = _load(d, "h0", heads, 1)
    dht = _load(d, "dht", heads, 1)
    ref = OB.chunk_gated_delta_rule_bwd(x["q"], x["k"], x["v"], x["g"], x["beta"], x["do"], dht=dht,
                                        initial_state=h0, **kw)
    out = {}
    for n, r in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), ref):
        if r is not None:
            out[n] = _sums(_load(d, n, heads, 1 if n == "dh0" else 2), r)
    return out


def fp8_frame_job(args):
    """One (frame, head group) of the streaming fp8 rollout: the frame's inputs are
    drawn again from their seed, q and k quantised and decoded as the test did, and the oracle runs from
    the state the HIP path started the frame with."""
    d, (f, heads), kw = args
    from oracle import gdn_oracle as O
    from gdn_inputs import dequant_bf16, make_inputs, quantize_fp8
    B, Tf, H, K, V = kw["shape"]
    x = make_inputs(B, Tf, H, K, V, seed=(kw["seed"], f), dtype="bf16", h0_scale=0.0)
    qc, qs = quantize_fp8(x["q"])
    kc, ks = quantize_fp8(x["k"])
    qd, kd = dequant_bf16(qc, qs), dequant_bf16(kc, ks)
    o_r, s_r = O.chunk_gated_delta_rule(qd[:, :, heads], kd[:, :, heads], x["v"][:, :, heads], x["g"][:, :, heads],
                                        x["beta"][:, :, heads], initial_state=_load(d, f"si{f}", heads, 1),
                                        output_final_state=True, dtype="bf16")
    return {f"o{f}": _sums(_load(d, f"o{f}", heads, 2), o_r), f"h{f}": _sums(_load(d, f"so{f}", heads, 1), s_r)}


def _combine(parts):
    tot = {}
    for p in parts:
        for n, (d2, r2, cnt) in p.items():
            a = tot.setdefault(n, [0.0, 0.0, 0])
            a[0] += d2
            a[1] += r2
            a[2] += cnt
    # RMS(x - ref) / (RMS(ref) + 1e-8), fla's get_err_ratio over all heads
    return {n: math.sqrt(d2 / cnt) / (math.sqrt(r2 / cnt) + 1e-8) for n, (d2, r2, cnt) in tot.items()}


def run_heads(job, scratch: Scratch, H: int, group: int, workers: int, kw: dict, log=print, frames: int = 0):
    """job over heads 0..H-1 in groups of ``group`` (and, with frames > 0, over (frame, group) pairs),
    ``workers`` child processes; returns the relative L2 error per output over all heads."""
    groups = [list(range(h, min(h + group, H))) for h in range(0, H, group)]
    items = [(f, hs) for f in range(frames) for hs in groups] if frames else groups
    ctx = mp.get_context("spawn")
    parts = []
    # one BLAS thread per child: the children already use the cores, and nested thread pools would
    # oversubscribe them many times over
    saved = {v: os.environ.get(v) for v in _THREAD_VARS}
    os.environ.update({v: "1" for v in _THREAD_VARS})
    try:
        with ProcessPoolExecutor(max_workers=min(workers, len(items)), mp_context=ctx) as ex:
            futs = {ex.submit(job, (scratch.path, it, kw)): it for it in items}
            for fut in as_completed(futs):
                it = futs[fut]
                hs = it[1] if frames else it
                parts.append(fut.result())
                log(f"    oracle on heads {hs[0]}..{hs[-1]}" + (f" of frame {it[0]}" if frames else "")
                    + f" done ({len(parts)} of {len(items)})")
    finally:
        for v, val in saved.items():
            if val is None:
                os.environ.pop(v, None)
            else:
                os.environ[v] = val
    return _combine(parts)


def forward_all_heads(x: dict, o, ht, dtype: str, workers: int = 8, group: int = 2, log=print, **kw):
    """Relative L2 of the HIP forward's o (and ht) against the oracle on every head.

    x: the numpy inputs (make_inputs); o [B, T, H, V], ht [N, H, K, V] or None as numpy float32
    (o bf16-valued when dtype is bf16)."""
    H = x["q"].shape[2]
    bf = dtype == "bf16"
    with Scratch() as s:
        for n in ("q", "k", "v"):
            s.put(n, x[n], bf16=bf)
        s.put("g", x["g"])
        s.put("beta", x["beta"], bf16=bf and x["beta"].dtype == np.float32 and _is_bf16(x["beta"]))
        s.put("h0", x.get("h0"))
        s.put("o", o, bf16=bf)
        s.put("ht", ht)
        return run_heads(_fwd_job, s, H, group, workers, dict(dtype=dtype, **kw), log=log)


def backward_all_heads(x: dict, do, dht, grads: dict, dtype: str, workers: int = 8, group: int = 2, log=print,
                       **kw):
    """Relative L2 of the HIP backward's gradients (dict dq, dk, dv, dg, dbeta, dh0 as numpy float32)
    against the backward oracle on every head."""
    H = x["q"].shape[2]
    bf = dtype == "bf16"
    with Scratch() as s:
        for n in ("q", "k", "v"):
            s.put(n, x[n], bf16=bf)
        s.put("g", x["g"])
        s.put("beta", x["beta"], bf16=bf and _is_bf16(x["beta"]))
        s.put("h0", x.get("h0"))
        s.put("do", do, bf16=bf)
        s.put("dht", dht)
        for n, a in grads.items():
            s.put(n, a)
        return run_heads(_bwd_job, s, H, group, workers, dict(dtype=dtype, **kw), log=log)


def _is_bf16(a) -> bool:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    return not np.any(u & 0xFFFF)
