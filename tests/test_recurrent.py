"""Short-sequence mode (fused_recurrent_gated_delta_rule, fla ops/gated_delta_rule/fused_recurrent.py).

CPU: pins the oracle's ``fused_recurrent`` against the fp64 token recurrence
(itself pinned against the chunked form), closed forms of each optional decay
and beta form, grouped value heads and the in-kernel L2 norm, and planted
mistakes.  GPU (``-m gpu``): the HIP kernel against that oracle through the C
ABI.  Tolerances (relative L2): fp32 inputs 1e-5 on o and final_state; bf16
inputs 1e-2 on o (one bf16 rounding of o) and 1e-5 on the fp32 final_state.
"""
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O
from gdn_inputs import make_inputs

rel = O.rel_l2


def case(B, T, H, K, V, seed, HV=None, cu=None, h0=0.5, dtype="fp32"):
    HV = HV or H
    rng = np.random.default_rng(seed)
    f32 = np.float32

    def unit(shape):
        x = rng.standard_normal(shape).astype(f32)
        return x / np.linalg.norm(x, axis=-1, keepdims=True)
    N = len(cu) - 1 if cu is not None else B
    x = dict(q=O.cast(unit((B, T, H, K)), dtype), k=O.cast(unit((B, T, H, K)), dtype),
             v=O.cast(rng.standard_normal((B, T, HV, V)).astype(f32), dtype),
             g=(-np.logaddexp(0, rng.standard_normal((B, T, HV)))).astype(f32),
             beta=O.cast(1 / (1 + np.exp(-rng.standard_normal((B, T, HV)))), dtype).astype(f32),
             h0=(h0 * rng.standard_normal((N, HV, K, V))).astype(f32) if h0 else None)
    return x


def fr(x, dtype="fp64", **kw):
    args = dict(g=x["g"], beta=x["beta"], initial_state=x["h0"])
    args.update(kw)
    return O.fused_recurrent(x["q"], x["k"], x["v"], dtype=dtype, **args)


# ---------------------------------------------------------------------------
# oracle pinning (CPU)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("cu", [None, np.array([0, 1, 40, 90])])
def test_scalar_gate_equals_token_recurrence(cu):
    x = case(1 if cu is not None else 2, 90, 3, 16, 8, seed=1, cu=cu)
    o, ht = fr(x, cu_seqlens=cu)
    on, hn = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"], cu_seqlens=cu)
    assert rel(o, on) < 1e-12 and rel(ht, hn) < 1e-12
    # and the fp32 mode (the kernel's arithmetic) stays close to fp64
    o32, h32 = fr(x, dtype="fp32", cu_seqlens=cu)
    assert rel(o32, on) < 1e-5 and rel(h32, hn) < 1e-5


def test_gk_and_gv_broadcast_of_g_equal_the_g_path():
    x = case(1, 40, 2, 16, 12, seed=2)
    o, ht = fr(x)
    gk = np.repeat(x["g"][..., None], 16, axis=-1)
    gv = np.repeat(x["g"][..., None], 12, axis=-1)
    ok_, hk = fr(x, g=None, gk=gk)
    ov, hv = fr(x, g=None, gv=gv)
    assert rel(ok_, o) < 1e-12 and rel(hk, ht) < 1e-12
    assert rel(ov, o) < 1e-12 and rel(hv, ht) < 1e-12


def test_beta_zero_closed_forms_of_gk_and_gv():
    x = case(1, 20, 2, 8, 6, seed=3)
    rng = np.random.default_rng(3)
    gk = -rng.random((1, 20, 2, 8))
    gv = -rng.random((1, 20, 2, 6))
    zero = np.zeros_like(x["beta"])
    _, hk = fr(x, g=None, gk=gk, beta=zero)
    np.testing.assert_allclose(hk[0], np.exp(gk.sum(1))[0][:, :, None] * x["h0"][0], rtol=1e-12)
    _, hv = fr(x, g=None, gv=gv, beta=zero)
    np.testing.assert_allclose(hv[0], x["h0"][0] * np.exp(gv.sum(1))[0][:, None, :], rtol=1e-12)
    # and o_t = scale q_t^T S_t with S_t the decayed state
    ok_, _ = fr(x, g=None, gk=gk, beta=zero)
    S3 = np.exp(gk[0, :4].sum(0))[:, :, None] * x["h0"][0]
    np.testing.assert_allclose(ok_[0, 3], 8 ** -0.5 * np.einsum("hkv,hk->hv", S3, x["q"][0, 3]), rtol=1e-10)


def test_per_column_beta():
    x = case(1, 30, 2, 8, 6, seed=4)
    o, ht = fr(x)
    bcol = np.repeat(x["beta"][..., None], 6, axis=-1)
    oc, hc = fr(x, beta=bcol)
    assert rel(oc, o) < 1e-12 and rel(hc, ht) < 1e-12
    # one token from a zero state: S = k (beta * v)^T, o = scale (q.k) beta * v
    y = case(1, 1, 2, 8, 6, seed=5, h0=0.0)
    b = np.random.default_rng(5).random((1, 1, 2, 6))
    o1, h1 = fr(y, g=None, beta=b)
    S = y["k"][0, 0].astype(np.float64)[:, :, None] * (b[0, 0] * y["v"][0, 0])[:, None, :]
    np.testing.assert_allclose(h1[0], S, rtol=1e-12)
    qk = np.sum(y["q"][0, 0].astype(np.float64) * y["k"][0, 0], -1)
    np.testing.assert_allclose(o1[0, 0], 8 ** -0.5 * qk[:, None] * b[0, 0] * y["v"][0, 0], rtol=1e-10, atol=1e-14)


def test_grouped_value_heads_equal_repeated_qk():
    x = case(1, 25, 2, 8, 8, seed=6, HV=6)
    o, ht = fr(x)
    xr = dict(x, q=np.repeat(x["q"], 3, axis=2), k=np.repeat(x["k"], 3, axis=2))
    o2, h2 = fr(xr)
    assert rel(o, o2) < 1e-12 and rel(ht, h2) < 1e-12
    # value head 1 uses q/k head 0 (not head 1): differs from a tiled mapping
    xt = dict(x, q=np.tile(x["q"], (1, 1, 3, 1)), k=np.tile(x["k"], (1, 1, 3, 1)))
    o3, _ = fr(xt)
    assert rel(o, o3) > 1e-2


def test_l2norm_in_kernel_equals_normalised_inputs():
    x = case(1, 30, 2, 16, 8, seed=7)
    xs = dict(x, q=x["q"] * 3.0, k=x["k"] * 0.25)
    o, ht = fr(xs, use_qk_l2norm_in_kernel=True)
    norm = lambda a: a / np.sqrt((a.astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-6)   # noqa: E731
    o2, h2 = fr(dict(x, q=norm(xs["q"]), k=norm(xs["k"])))
    assert rel(o, o2) < 1e-12 and rel(ht, h2) < 1e-12


def _gk_over_v(f, g_t, gk_t, gv_t, HV, K, V):
    d = _orig_decay(f, g_t, None, gv_t, HV, K, V)
    return d if gk_t is None else d * np.exp(np.asarray(gk_t, f))[:, None, :]   # K == V here


def _decay_after_delta(S, decay, qt, kt, vt, bt):
    vp = bt * (vt - np.sum(S * kt[:, :, None], axis=1))
    S = (S + kt[:, :, None] * vp[:, None, :]) * decay
    return S, np.sum(S * qt[:, :, None], axis=1)


def _tiled_heads(x, rep):
    return np.tile(x, (1, 1, rep, 1))


_orig_decay = O._rec_decay


@pytest.mark.parametrize("target,replacement", [
    ("_rec_decay", _gk_over_v), ("_rec_token", _decay_after_delta), ("_rec_heads", _tiled_heads)])
def test_planted_mistake_is_caught(monkeypatch, target, replacement):
    x = case(1, 30, 2, 8, 8, seed=8, HV=4)
    gk = -np.random.default_rng(8).random((1, 30, 4, 8))
    ref = dict(gk=gk)
    o_good, _ = fr(x, **ref)
    # the good oracle's gk path agrees with its closed form above; the planted one must not agree with it
    monkeypatch.setattr(O, target, replacement)
    o_bad, _ = fr(x, **ref)
    monkeypatch.undo()
    assert rel(o_bad, o_good) > 1e-3


# ---------------------------------------------------------------------------
# GPU parity through the C ABI
# ---------------------------------------------------------------------------
GPU_CASES = [
    # id, B, T, H, HV, K, V, cu, dtype, extras
    ("decode_cfg4", 8, 1, 20, 20, 128, 128, None, "bf16", ""),
    ("t64_varlen", 1, 130, 4, 4, 128, 128, [0, 1, 64, 130], "bf16", ""),
    ("model_shape", 2, 3, 4, 4, 256, 512, None, "bf16", "l2"),
    ("gva_fp32", 2, 20, 2, 6, 64, 48, None, "fp32", ""),
    ("gk_gv_colbeta", 1, 33, 3, 3, 32, 40, None, "fp32", "gk,gv,colbeta"),
    ("k16_v_ragged", 3, 9, 2, 2, 16, 20, None, "bf16", "nobeta"),
    ("no_h0_no_g", 1, 17, 2, 2, 128, 64, None, "bf16", "nog,noh0"),
    # the vector form (K in {64, 128, 256}, V a multiple of 16) with every optional input
    ("vec_gk_gv_colbeta", 2, 21, 2, 4, 64, 32, None, "fp32", "gk,gv,colbeta"),
    ("vec_varlen_k256", 1, 40, 2, 2, 256, 64, [0, 7, 7, 40], "bf16", "l2"),
]


def _random_gpu_cases(n=12, seed=20265):
    """Seeded random draws over the same space: K in {16, .., 256} (the vector form where K is 64, 128
    or 256 and V a multiple of 16, the scalar form otherwise), ragged V, grouped value heads, batch or
    varlen (with an empty sequence), and the optional gates, per-column beta, no beta, no g, no initial
    state and the L2 norm."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        K = int(rng.choice([16, 32, 64, 128, 256]))
        V = int(rng.choice([16, 40, 64, 128])) if K < 256 else int(rng.choice([64, 128]))
        H = int(rng.integers(1, 4))
        HV = H * int(rng.choice([1, 2]))
        dt = "fp32" if rng.random() < 0.3 else "bf16"
        if rng.random() < 0.35:
            lens = [int(x) for x in rng.integers(1, 50, int(rng.integers(2, 5)))]
            lens[int(rng.integers(0, len(lens)))] = 0
            B, T, cu = 1, sum(lens), [0] + [int(x) for x in np.cumsum(lens)]
        else:
            B, T, cu = int(rng.integers(1, 5)), int(rng.integers(1, 40)), None
        extras = [e for e, p_ in (("gk", 0.3), ("gv", 0.3), ("colbeta", 0.25), ("nog", 0.15), ("noh0", 0.2),
                                  ("l2", 0.3)) if rng.random() < p_]
        if "colbeta" not in extras and rng.random() < 0.1:
            extras.append("nobeta")
        out.append((f"rand{i:02d}", B, T, H, HV, K, V, cu, dt, ",".join(extras)))
    return out


GPU_CASES += _random_gpu_cases()


@pytest.mark.gpu
@pytest.mark.parametrize("cid,B,T,H,HV,K,V,cu,dt,extras", GPU_CASES, ids=[c[0] for c in GPU_CASES])
def test_gpu_fused_recurrent(cid, B, T, H, HV, K, V, cu, dt, extras):
    import torch
    import kairos_gdn
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print(f"fused_recurrent {cid}: B={B} T={T} H={H} HV={HV} K={K} V={V} cu={cu} {dt} {extras}", flush=True)
    sys.stdout.flush()
    cu_np = np.array(cu) if cu else None
    x = case(B, T, H, K, V, seed=K + V + T, HV=HV, cu=cu_np, h0=0.0 if "noh0" in extras else 0.5, dtype=dt)
    rng = np.random.default_rng(T)
    ex = {}
    if "gk" in extras:
        ex["gk"] = (-rng.random((B, T, HV, K)) * 0.2).astype(np.float32)
    if "gv" in extras:
        ex["gv"] = (-rng.random((B, T, HV, V)) * 0.2).astype(np.float32)
    beta = x["beta"]
    if "colbeta" in extras:                  # in the call's dtype, as the kernel receives it
        beta = O.cast(rng.random((B, T, HV, V)).astype(np.float32), dt)
    if "nobeta" in extras:
        beta = None
    g = None if "nog" in extras else x["g"]
    l2 = "l2" in extras
    if l2:
        x["q"] = O.cast(x["q"] * 2.0, dt)
        x["k"] = O.cast(x["k"] * 0.5, dt)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    d = lambda a, t=torch.float32: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda", t)  # noqa
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    o, ht = kairos_gdn.fused_recurrent_gated_delta_rule(
        d(x["q"], tdt), d(x["k"], tdt), d(x["v"], tdt), g=d(g), gk=d(ex.get("gk")), gv=d(ex.get("gv")),
        beta=d(beta, tdt) if beta is not None else None, initial_state=d(x["h0"]), output_final_state=True,
        use_qk_l2norm_in_kernel=l2, cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert o.dtype == tdt and tuple(o.shape) == (B, T, HV, V) and ht.dtype == torch.float32
    o_r, ht_r = O.fused_recurrent(x["q"], x["k"], x["v"], g=g, gk=ex.get("gk"), gv=ex.get("gv"), beta=beta,
                                  initial_state=x["h0"], cu_seqlens=cu_np, use_qk_l2norm_in_kernel=l2,
                                  dtype="fp32", o_dtype=dt)
    eo = rel(o.float().cpu().numpy(), o_r)
    eh = rel(ht.cpu().numpy(), ht_r)
    print(f"    rel-L2 o={eo:.3e} final_state={eh:.3e}", flush=True)
    assert eo < (1e-2 if dt == "bf16" else 1e-5)
    assert eh < 1e-5


@pytest.mark.gpu
def test_gpu_fused_recurrent_matches_chunked_op():
    """T <= 64: the layer switches between the two ops; both must give the same result."""
    import torch
    import kairos_gdn
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("fused_recurrent vs chunk_gated_delta_rule, T=64", flush=True)
    x = make_inputs(2, 64, 4, 128, 128, seed=11, dtype="bf16")
    d = lambda a, t: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", t)  # noqa: E731
    bf = torch.bfloat16
    # keywords: the two ops order their optional arguments differently (fused_recurrent takes gk, gv before beta)
    args = dict(q=d(x["q"], bf), k=d(x["k"], bf), v=d(x["v"], bf), g=d(x["g"], torch.float32), beta=d(x["beta"], bf),
                initial_state=d(x["h0"], torch.float32), output_final_state=True)
    o1, h1 = kairos_gdn.fused_recurrent_gated_delta_rule(**args)
    o2, h2 = kairos_gdn.chunk_gated_delta_rule(**args)
    torch.cuda.synchronize()
    eo = rel(o1.float().cpu().numpy(), o2.float().cpu().numpy())
    eh = rel(h1.cpu().numpy(), h2.cpu().numpy())
    print(f"    rel-L2 o={eo:.3e} final_state={eh:.3e}", flush=True)
    assert eo < 1e-2 and eh < 5e-3
