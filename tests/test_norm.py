"""Gated RMSNorm, the GatedDeltaNet layer's output epilogue (fla modules/fused_norm_gate.py).

CPU: the oracle (oracle/gdn_oracle.py: rms_norm_gated) is pinned against
torch.nn.functional.rms_norm times silu / sigmoid of the gate in fp64 (library
routines) and against closed forms; the host layer mirrors the reference's
module and argument errors.  GPU (-m gpu): the HIP kernel behind
kairos_gdn_rms_norm_gated against the oracle.

Tolerances: fp32 output rtol 1e-5; bf16 output at most one bf16 ulp from the
oracle's rounded value (both compute in fp32 and round once), with at least 99%
of elements identical.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn_oracle as O


def _rows(rows, D, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, D)) * rng.uniform(0.1, 3.0, (rows, 1))
    g = rng.standard_normal((rows, D)) * 2.0
    w = rng.uniform(0.5, 1.5, D)
    b = rng.standard_normal(D) * 0.1
    return x, g, w, b


@pytest.mark.parametrize("activation", ["swish", "silu", "sigmoid"])
@pytest.mark.parametrize("affine", [(True, False), (True, True), (False, False)])
def test_oracle_against_torch_rms_norm(activation, affine):
    x, g, w, b = _rows(33, 128, seed=1)
    w = w if affine[0] else None
    b = b if affine[1] else None
    eps = 1e-5
    y, rstd = O.rms_norm_gated(x, g, w, b, activation, eps, dtype="fp64")
    xt, gt = torch.from_numpy(x), torch.from_numpy(g)
    ref = F.rms_norm(xt, (128,), weight=None if w is None else torch.from_numpy(w), eps=eps)
    if b is not None:
        ref = ref + torch.from_numpy(b)
    ref = ref * (F.silu(gt) if activation != "sigmoid" else torch.sigmoid(gt))
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(rstd, torch.rsqrt(xt.pow(2).mean(-1) + eps).numpy(), rtol=1e-12)


def test_oracle_closed_forms():
    D, eps = 64, 1e-6
    x, g, w, _ = _rows(5, D, seed=2)
    zero = np.zeros_like(g)
    y, rstd = O.rms_norm_gated(x, zero, w, None, "swish", eps, dtype="fp64")
    np.testing.assert_array_equal(y, 0.0)                       # silu(0) = 0
    y, _ = O.rms_norm_gated(x, zero, w, None, "sigmoid", eps, dtype="fp64")
    np.testing.assert_allclose(y, 0.5 * x * rstd[:, None] * w, rtol=1e-12)
    c = np.full((1, D), -2.5)                                   # constant row
    y, _ = O.rms_norm_gated(c, np.full((1, D), 40.0), None, None, "sigmoid", eps, dtype="fp64")
    np.testing.assert_allclose(y, -2.5 / np.sqrt(6.25 + eps) / (1.0 + np.exp(-40.0)), rtol=1e-12)
    y1, _ = O.rms_norm_gated(x, g, w, None, "swish", 0.0, dtype="fp64")
    y2, _ = O.rms_norm_gated(7.0 * x, g, w, None, "swish", 0.0, dtype="fp64")
    np.testing.assert_allclose(y1, y2, rtol=1e-12)              # scale invariance at eps = 0


def test_oracle_planted_mistake_fails():
    """A norm over the sum instead of the mean (a plausible slip) is caught by the library check."""
    x, g, w, _ = _rows(4, 128, seed=3)
    y, _ = O.rms_norm_gated(x, g, w, None, "swish", 1e-5, dtype="fp64")
    wrong = x / np.sqrt(np.sum(x * x, -1, keepdims=True) + 1e-5) * w * g / (1 + np.exp(-g))
    assert not np.allclose(y, wrong, rtol=1e-3)


def test_oracle_bf16_storage_rounds_once():
    x, g, w, _ = _rows(8, 128, seed=4)
    x, g = O.to_bf16(x.astype(np.float32)), O.to_bf16(g.astype(np.float32))
    y16, _ = O.rms_norm_gated(x, g, w, None, "swish", 1e-5, dtype="bf16")
    y32, _ = O.rms_norm_gated(x, g, w, None, "swish", 1e-5, dtype="fp32")
    np.testing.assert_array_equal(y16, O.to_bf16(y32))


def test_module_mirrors_reference_interface():
    import kairos_gdn
    m = kairos_gdn.FusedRMSNormGated(128, eps=1e-5)
    assert repr(m) == "FusedRMSNormGated(128, eps=1e-05, activation=swish)"
    assert m.weight.shape == (128,) and torch.all(m.weight == 1) and m.bias is None
    m2 = kairos_gdn.FusedRMSNormGated(64, elementwise_affine=False, activation="sigmoid")
    assert m2.weight is None and "elementwise_affine=False" in repr(m2)
    with pytest.raises(ValueError, match="Unsupported activation"):
        kairos_gdn.FusedRMSNormGated(64, activation="relu")


def test_host_errors_and_no_cpu_path():
    import kairos_gdn
    x = torch.zeros(4, 64)
    with pytest.raises(NotImplementedError):
        kairos_gdn.rms_norm_gated(x, x, None, None, residual=x)
    with pytest.raises(ValueError, match="Unsupported activation"):
        kairos_gdn.rms_norm_gated_fwd(x, x, None, None, activation="gelu")
    with pytest.raises(ValueError, match="gate shape"):
        kairos_gdn.rms_norm_gated_fwd(x, x[:2], None, None)
    with pytest.raises(RuntimeError, match="HIP device only"):
        kairos_gdn.rms_norm_gated_fwd(x, x, None, None)


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------
def _check(y, y_ref, dt):
    y = y.float().cpu().numpy()
    if dt == torch.float32:
        np.testing.assert_allclose(y, y_ref, rtol=1e-5, atol=1e-6)
        return
    ulp = np.maximum(np.abs(y_ref), 1e-30) * 2.0 ** -7
    diff = np.abs(y - y_ref)
    assert np.all(diff <= ulp + 1e-30), float(np.max(diff / ulp))
    assert np.mean(diff == 0) >= 0.99


@pytest.mark.gpu
@pytest.mark.parametrize("rows,D", [(1, 128), (37, 64), (1000, 96), (2049, 128), (300, 256), (130, 512), (5, 8)])
@pytest.mark.parametrize("xdt,gdt", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.float32)])
def test_rms_norm_gated_gpu(rows, D, xdt, gdt):
    import kairos_gdn
    print(f"rms_norm_gated rows={rows} D={D} x={xdt} g={gdt}", flush=True)
    x, g, w, b = _rows(rows, D, seed=rows + D)
    xt = torch.from_numpy(x).to(xdt)
    gt = torch.from_numpy(g).to(gdt)
    wt = torch.from_numpy(w).float()
    sdt = "bf16" if xdt == torch.bfloat16 else "fp32"
    for act, use_w, use_b, eps in [("swish", True, False, 1e-5), ("sigmoid", True, True, 1e-6),
                                   ("silu", False, False, 1e-5)]:
        y, rstd = kairos_gdn.rms_norm_gated_fwd(xt.cuda(), gt.cuda(), wt.cuda() if use_w else None,
                                                torch.from_numpy(b).float().cuda() if use_b else None,
                                                act, eps, return_rstd=True)
        torch.cuda.synchronize()
        assert y.dtype == xdt and y.shape == xt.shape
        y_ref, r_ref = O.rms_norm_gated(xt.float().numpy(), gt.float().numpy(), w if use_w else None,
                                        b if use_b else None, act, eps, dtype=sdt)
        _check(y, y_ref, xdt)
        np.testing.assert_allclose(rstd.cpu().numpy(), r_ref, rtol=1e-5)


@pytest.mark.gpu
def test_module_on_layer_shape_gpu():
    """FusedRMSNormGated(head_v_dim) on o-shaped input [B, T, H, V], bf16 weight, as the layer applies it."""
    import kairos_gdn
    print("FusedRMSNormGated [2, 300, 4, 128] bf16", flush=True)
    m = kairos_gdn.FusedRMSNormGated(128, eps=1e-5).cuda().to(torch.bfloat16)
    with torch.no_grad():
        m.weight.copy_(torch.linspace(0.5, 1.5, 128))
    x, g, _, _ = _rows(2 * 300 * 4, 128, seed=9)
    xt = torch.from_numpy(x).to(torch.bfloat16).reshape(2, 300, 4, 128)
    gt = torch.from_numpy(g).to(torch.bfloat16).reshape(2, 300, 4, 128)
    with torch.no_grad():
        y = m(xt.cuda(), gt.cuda())
    torch.cuda.synchronize()
    y_ref, _ = O.rms_norm_gated(xt.float().numpy(), gt.float().numpy(), m.weight.detach().float().cpu().numpy(), None,
                                "swish", 1e-5, dtype="bf16")
    _check(y, y_ref, torch.bfloat16)
