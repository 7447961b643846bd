"""GPU parity of the forward with the layer's prologue folded in (kairos_gdn_chunk_fwd_conv).

The reference layer runs three ShortConvolutions (kernel size 4, SiLU) on the q/k/v projections and
then chunk_gated_delta_rule (fla layers/gated_deltanet.py:234-285).  Each case here runs the fused
call through the C ABI and compares it with the oracle's composition of the same two steps
(O.causal_conv1d on each projection, then O.chunk_gated_delta_rule), including the conv caches in
and out and packed variable-length batches: o and final_state within the north-star tolerances
(rel-L2 1e-2 / 5e-3), the caches bit for bit.  Without the L2 norm the fused call also equals the
two-step HIP path (kairos_gdn.causal_conv1d, then kairos_gdn.chunk_gated_delta_rule) bit for bit: the
folded convolution is the standalone kernel's arithmetic.
"""
import numpy as np
import pytest
import torch

import kairos_gdn
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def note(msg):
    print(msg, flush=True)


def make_case(B, T, H, K, V, seed, cu=None, cache=True, bias=False, wdt="bf16", h0=True, l2=True):
    """Projections ~ N(0, 1), taps ~ N(0, s^2): with the in-op L2 norm s = 0.5; without it the keys are
    used as they come, so s = K^-1/2 keeps |k| near 1 (beta |k|^2 < 2, the delta rule's stable range)."""
    rng = np.random.default_rng(seed)
    s_w = 0.5 if l2 else K ** -0.5
    N = len(cu) - 1 if cu else B
    f32 = np.float32
    x = {}
    for n, D in (("q", H * K), ("k", H * K), ("v", H * V)):
        x["x" + n] = O.to_bf16(rng.standard_normal((B, T, D), dtype=f32))
        x["w" + n] = O.cast((s_w * rng.standard_normal((D, 4))).astype(f32), wdt)
        x["b" + n] = O.cast((0.1 * rng.standard_normal(D)).astype(f32), wdt) if bias else None
        x["c" + n] = O.to_bf16(rng.standard_normal((N, D, 4), dtype=f32)) if cache else None
    x["g"] = (-np.logaddexp(0.0, rng.standard_normal((B, T, H), dtype=f32))).astype(f32)
    x["beta"] = O.to_bf16(1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H), dtype=f32))))
    x["h0"] = (0.02 * rng.standard_normal((N, H, K, V), dtype=f32)).astype(f32) if h0 else None
    x["shape"] = (B, T, H, K, V)
    x["cu"] = cu
    return x


def oracle_conv(x):
    B, T, H, K, V = x["shape"]
    cu = np.array(x["cu"]) if x["cu"] else None
    y, caches = {}, {}
    for n in ("q", "k", "v"):
        y[n], caches[n] = O.causal_conv1d(x["x" + n], x["w" + n], x["b" + n], initial_state=x["c" + n],
                                          cu_seqlens=cu, activation="silu", dtype="bf16")
    return (y["q"].reshape(B, T, H, K), y["k"].reshape(B, T, H, K), y["v"].reshape(B, T, H, V)), caches


def run_fused(x, l2, wdt="bf16"):
    tw = torch.bfloat16 if wdt == "bf16" else torch.float32
    d = lambda a, dt=torch.bfloat16: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)  # noqa: E731
    cu_t = torch.tensor(x["cu"], dtype=torch.int64, device="cuda") if x["cu"] else None
    o, ht, caches = kairos_gdn.chunk_gated_delta_rule_conv(
        d(x["xq"]), d(x["xk"]), d(x["xv"]), d(x["g"], torch.float32), d(x["beta"]), d(x["wq"], tw), d(x["wk"], tw),
        d(x["wv"], tw), d(x["bq"], tw), d(x["bk"], tw), d(x["bv"], tw), initial_state=d(x["h0"], torch.float32),
        output_final_state=True, conv_state=(d(x["cq"]), d(x["ck"]), d(x["cv"])), output_conv_state=True,
        cu_seqlens=cu_t, use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    return o, ht, caches


CASES = [
    # name, shape (B, T, H, K, V), cu, cache, bias, weight dtype, l2
    ("layer dims, caches, L2", (1, 300, 2, 256, 512), None, True, False, "bf16", True),
    ("layer dims, no caches", (1, 300, 2, 256, 512), None, False, False, "bf16", False),
    ("layer dims, pipelined parts, bias, fp32 taps, L2", (1, 1100, 2, 256, 512), None, True, True, "fp32", True),
    ("layer dims varlen with a 1-token and a 3-token sequence", (1, 400, 2, 256, 256), [0, 1, 4, 130, 400], True,
     False, "bf16", True),
    ("layer dims batch 2 ragged, 3 value tiles", (2, 150, 3, 256, 192), None, True, False, "bf16", False),
    ("dk = dv = 128 (the convolution ahead of the segment scan)", (1, 500, 2, 128, 128), [0, 2, 200, 500], True,
     True, "bf16", True),
]


@pytest.mark.parametrize("name,shape,cu,cache,bias,wdt,l2", CASES, ids=[c[0] for c in CASES])
def test_fused_conv_against_oracle(name, shape, cu, cache, bias, wdt, l2):
    B, T, H, K, V = shape
    note(f"fused prologue {name}: B={B} T={T} H={H} K={K} V={V} cu={cu} cache={cache} bias={bias} {wdt} l2={l2}")
    x = make_case(B, T, H, K, V, seed=T + K + V, cu=cu, cache=cache, bias=bias, wdt=wdt, l2=l2)
    o, ht, caches = run_fused(x, l2, wdt)
    (q, k, v), c_ref = oracle_conv(x)
    o_r, ht_r = O.chunk_gated_delta_rule(q, k, v, x["g"], x["beta"], initial_state=x["h0"], output_final_state=True,
                                         cu_seqlens=np.array(cu) if cu else None, use_qk_l2norm_in_kernel=l2,
                                         dtype="bf16")
    eo = O.rel_l2(o.float().cpu().numpy(), o_r)
    eh = O.rel_l2(ht.cpu().numpy(), ht_r)
    note(f"    rel-L2 o={eo:.3e} final_state={eh:.3e}")
    assert eo < 1e-2 and eh < 5e-3
    for i, n in enumerate(("q", "k", "v")):
        np.testing.assert_array_equal(caches[i].float().cpu().numpy(), c_ref[n])


@pytest.mark.parametrize("shape,cu", [((1, 700, 2, 256, 512), None), ((1, 400, 2, 256, 256), [0, 1, 4, 130, 400])])
def test_fused_conv_equals_two_step_bit_for_bit(shape, cu):
    """Without the L2 norm the fused call gives the bits of causal_conv1d on each projection followed by
    chunk_gated_delta_rule (both through this library's kernels)."""
    B, T, H, K, V = shape
    note(f"fused prologue vs two-step HIP path: {shape} cu={cu}")
    x = make_case(B, T, H, K, V, seed=7 + T, cu=cu, cache=True, bias=True, l2=False)
    o, ht, caches = run_fused(x, False)
    d = lambda a, dt=torch.bfloat16: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)  # noqa: E731
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    ys = []
    for n, dh in (("q", K), ("k", K), ("v", V)):
        y, c = kairos_gdn.causal_conv1d(d(x["x" + n]), d(x["w" + n]), d(x["b" + n]), initial_state=d(x["c" + n]),
                                        output_final_state=True, activation="silu", cu_seqlens=cu_t)
        ys.append(y.view(B, T, H, dh))
        assert torch.equal(c, caches[("q", "k", "v").index(n)])
    o2, ht2 = kairos_gdn.chunk_gated_delta_rule(ys[0], ys[1], ys[2], d(x["g"], torch.float32), d(x["beta"]),
                                                initial_state=d(x["h0"], torch.float32), output_final_state=True,
                                                cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all()) and bool(torch.isfinite(ht).all())
    assert torch.equal(o, o2)
    assert torch.equal(ht, ht2)


def test_fused_conv_model_shape_full_size():
    """The Kairos layer at the headline clip length (T=32760, H=20, K=256, V=512), its own mode (in-op L2
    norm, conv caches in and out), against the oracle's composition on every head."""
    import oracle_pool
    B, T, H, K, V = 1, 32760, 20, 256, 512
    note(f"fused prologue, model shape B={B} T={T} H={H} K={K} V={V}, L2, caches (oracle on all heads)")
    x = make_case(B, T, H, K, V, seed=20273, cache=True)
    o, ht, caches = run_fused(x, True)
    note("    HIP call done; oracle convolution")
    (q, k, v), c_ref = oracle_conv(x)
    for i, n in enumerate(("q", "k", "v")):
        np.testing.assert_array_equal(caches[i].float().cpu().numpy(), c_ref[n])
    xo = dict(q=q, k=k, v=v, g=x["g"], beta=x["beta"], h0=x["h0"])
    e = oracle_pool.forward_all_heads(xo, o.float().cpu().numpy(), ht.cpu().numpy(), "bf16", workers=8, group=2,
                                      log=note, use_qk_l2norm_in_kernel=True)
    note(f"    rel-L2 over all heads o={e['o']:.3e} ht={e['ht']:.3e}")
    assert e["o"] < 1e-2 and e["ht"] < 5e-3
