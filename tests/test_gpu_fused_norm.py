"""The forward with the layer's gated RMSNorm (kairos_gdn_chunk_fwd_gated_norm).

y = o_norm(chunk_gated_delta_rule(...)[0], gate) (fla layers/gated_deltanet.py:275-311).  Each case
runs the plain forward for o, then the combined call, and checks:
  - y against the oracle's rms_norm_gated of that o (oracle/gdn_oracle.py, pinned in test_norm.py):
    every element within one bf16 ulp of the oracle's rounded value and at least 99% identical
    (both compute in fp32 and round once; the fused epilogue sums the squares in another order);
  - y against the oracle's whole layer (chunk_gated_delta_rule then rms_norm_gated on bf16 o):
    relative L2 <= 1e-2, the forward's own bar;
  - the separate-kernel form (KAIROS_GDN_FUSED_NORM=0) against the same oracle bar.
Cases cover the fused output kernel (bf16, head dims 64 / 128, bf16 gate), the fused K = 256 kernel
with the norm folded in (KAIROS_GDN_WIDE_NORM_FOLD=1: its workgroups of 64 value columns exchange
per-token sums of squares), ragged and varlen chunks,
the in-op L2 norm, and the forms that run the norm kernel after the output (fp32 gate, fp32 v).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
from gdn_inputs import make_inputs
import kairos_gdn

pytestmark = pytest.mark.gpu

TDT = {"bf16": torch.bfloat16, "fp32": torch.float32}


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype)


@pytest.fixture(scope="module", autouse=True)
def _gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    kairos_gdn._lib.load()


def _norm_params(V, seed, w_dtype):
    rng = np.random.default_rng(seed)
    w = rng.uniform(0.5, 1.5, V)
    b = rng.standard_normal(V) * 0.1
    wt = torch.from_numpy(w).to(w_dtype)
    bt = torch.from_numpy(b).to(w_dtype)
    return wt.float().numpy().astype(np.float64), bt.float().numpy().astype(np.float64), wt.cuda(), bt.cuda()


def _magnitude(x, g, w, b, act, eps):
    """(|x| rstd |w| + |b|) |act(g)| per element: the size of the terms whose fp32 rounding the
    kernel and the oracle order differently (a bias can cancel x rstd w, leaving y far smaller)."""
    m, _ = O.rms_norm_gated(np.abs(x), g, None if w is None else np.abs(w), None if b is None else np.abs(b),
                            act, eps, dtype="fp32")
    return np.abs(m)


def _within_ulp(y, y_ref, dt, mag=None):
    """|y - y_ref| <= one ulp of y_ref in y's storage dtype + 2^-20 mag (a few fp32 roundings of the
    terms before they cancel), and at least 99% of the elements identical."""
    y = y.float().cpu().numpy()
    slack = 0.0 if mag is None else mag * 2.0 ** -20
    if dt == "fp32":
        np.testing.assert_allclose(y, y_ref, rtol=2e-5, atol=1e-6)
        return
    ulp = np.maximum(np.abs(y_ref), 1e-30) * 2.0 ** -7
    diff = np.abs(y - y_ref)
    bad = diff > ulp + slack + 1e-30
    if np.any(bad):
        i = np.unravel_index(np.argmax(diff / (ulp + slack)), diff.shape)
        raise AssertionError(f"{int(bad.sum())} elements beyond the bar; worst at {i}: y={y[i]!r} "
                             f"ref={y_ref[i]!r} ulp={ulp[i]!r} slack={np.broadcast_to(slack, diff.shape)[i]!r}")
    assert np.mean(diff == 0) >= 0.99, float(np.mean(diff == 0))


CASES = [
    # dt, B, T, H, K, V, cu, l2, gate dtype, activation, weight (None / "f32" / "bf16"), bias
    ("bf16", 1, 1, 2, 128, 128, None, False, "bf16", "swish", "f32", False),
    ("bf16", 1, 700, 3, 128, 128, None, False, "bf16", "swish", "bf16", False),
    ("bf16", 2, 333, 2, 64, 64, None, False, "bf16", "sigmoid", "f32", True),
    ("bf16", 1, 700, 3, 64, 128, [0, 1, 1, 129, 640, 700], False, "bf16", "silu", None, False),
    ("bf16", 3, 200, 2, 128, 64, None, True, "bf16", "swish", "f32", True),
    ("bf16", 1, 4100, 4, 128, 128, [0, 63, 64, 65, 2000, 4100], True, "bf16", "swish", "bf16", True),
    # the fused K = 256 form (workgroups of 64 value columns exchange sums of squares): varlen with a
    # 1-token sequence, the pipelined parts (T = 700: 11 chunks in 4 parts), one value tile, one chunk
    ("bf16", 1, 400, 2, 256, 512, [0, 1, 130, 400], False, "bf16", "swish", "bf16", False),
    ("bf16", 1, 700, 2, 256, 512, None, True, "bf16", "swish", "f32", True),
    ("bf16", 2, 130, 3, 256, 64, None, False, "bf16", "sigmoid", None, False),
    ("bf16", 1, 64, 1, 256, 192, None, False, "bf16", "swish", "bf16", True),
    ("bf16", 1, 257, 2, 256, 256, [0, 1, 1, 200, 257], True, "bf16", "silu", "f32", False),
    # the norm kernel after the output: fp32 gate, K = 256 with an fp32 gate, fp32 v
    ("bf16", 1, 300, 2, 128, 128, None, False, "fp32", "swish", "f32", False),
    ("bf16", 1, 300, 2, 256, 512, None, False, "fp32", "swish", "f32", False),
    ("fp32", 2, 150, 2, 128, 64, None, False, "fp32", "sigmoid", "f32", True),
    # the pipelined K = 256 forward with the norm applied part by part: two sequences (one norm launch
    # per sequence and part), an fp32 gate
    ("bf16", 2, 600, 2, 256, 128, None, True, "bf16", "swish", "bf16", False),
    ("bf16", 1, 650, 2, 256, 512, None, False, "fp32", "swish", "f32", True),
]


@pytest.mark.parametrize("dt,B,T,H,K,V,cu,l2,gdt,act,wkind,use_b", CASES)
def test_gated_norm_forward(dt, B, T, H, K, V, cu, l2, gdt, act, wkind, use_b, monkeypatch):
    note(f"chunk_fwd_gated_norm {dt} B={B} T={T} H={H} K={K} V={V} cu={cu} l2={l2} gate={gdt} act={act} "
         f"w={wkind} b={use_b}")
    n = len(cu) - 1 if cu else None
    x = make_inputs(B, T, H, K, V, seed=T + 7 * H + K, dtype=dt, n_states=n, h0_scale=0.02)
    if l2:
        x["q"] = O.cast(x["q"] * 3.0, dt)
        x["k"] = O.cast(x["k"] * 0.5, dt)
    rng = np.random.default_rng(T + V)
    gate_np = rng.standard_normal((B, T, H, V)) * 2.0
    gate = dev(gate_np, torch.bfloat16 if gdt == "bf16" else torch.float32)
    gate_np = gate.float().cpu().numpy().astype(np.float64)
    w_np = b_np = w_t = b_t = None
    if wkind is not None or use_b:
        wd = torch.bfloat16 if wkind == "bf16" else torch.float32
        w_np, b_np, w_t, b_t = _norm_params(V, V, wd)
        if wkind is None:
            w_np, w_t = None, None
        if not use_b:
            b_np, b_t = None, None
    eps = 1e-5
    d = {k: dev(x[k], TDT[dt]) for k in ("q", "k", "v", "beta")}
    d["g"] = dev(x["g"])
    h0 = dev(x["h0"])
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu is not None else None
    o, ht = kairos_gdn.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=h0,
                                              output_final_state=True, cu_seqlens=cu_t,
                                              use_qk_l2norm_in_kernel=l2)
    o_np = o.float().cpu().numpy()
    y_ref, _ = O.rms_norm_gated(o_np.reshape(-1, V), gate_np.reshape(-1, V), w_np, b_np, act, eps, dtype=dt)
    y_ref = y_ref.reshape(B, T, H, V)
    mag = _magnitude(o_np.reshape(-1, V), gate_np.reshape(-1, V), w_np, b_np, act, eps).reshape(B, T, H, V)
    o_or, _ = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                       output_final_state=True, cu_seqlens=np.array(cu) if cu else None,
                                       use_qk_l2norm_in_kernel=l2, dtype=dt)
    y_layer, _ = O.rms_norm_gated(o_or.reshape(-1, V), gate_np.reshape(-1, V), w_np, b_np, act, eps, dtype=dt)
    for fused in ("1", "0", "fold"):
        # "1": the default (at K = 256 with pipelined parts the norm kernel part by part); "0": the norm
        # kernel over all rows after the forward; "fold": the K = 256 form's norm in the fused kernel
        # (opt-in), elsewhere as "1"
        monkeypatch.setenv("KAIROS_GDN_FUSED_NORM", "0" if fused == "0" else "1")
        monkeypatch.setenv("KAIROS_GDN_NORM_PARTS", "0" if fused == "0" else "1")
        monkeypatch.setenv("KAIROS_GDN_WIDE_NORM_FOLD", "1" if fused == "fold" else "0")
        y, ht2 = kairos_gdn.chunk_gated_delta_rule_gated_norm(
            d["q"], d["k"], d["v"], d["g"], d["beta"], gate, w_t, b_t, initial_state=h0, output_final_state=True,
            cu_seqlens=cu_t, use_qk_l2norm_in_kernel=l2, activation=act, eps=eps)
        torch.cuda.synchronize()
        assert y.dtype == TDT[dt] and tuple(y.shape) == (B, T, H, V)
        assert torch.equal(ht2, ht)
        _within_ulp(y, y_ref, dt, mag)
        e = O.rel_l2(y.float().cpu().numpy(), y_layer.reshape(B, T, H, V))
        note(f"    fused={fused} rel-L2 y vs the oracle layer = {e:.3e}")
        assert e < 1e-2


def test_gated_norm_config2_full_size(monkeypatch):
    """BASELINE config 2 (T=32760, H=20, d=128, bf16): the fused output kernel against the plain
    forward followed by the oracle's norm on every 97th token (size-independent: the norm is per row)."""
    B, T, H, K, V = 1, 32760, 20, 128, 128
    note(f"chunk_fwd_gated_norm full size B={B} T={T} H={H} K={K} V={V}")
    x = make_inputs(B, T, H, K, V, seed=5, dtype="bf16", h0_scale=0.02)
    d = {k: dev(x[k], torch.bfloat16) for k in ("q", "k", "v", "beta")}
    d["g"] = dev(x["g"])
    h0 = dev(x["h0"])
    gen = torch.Generator(device="cuda").manual_seed(3)
    gate = (torch.randn(B, T, H, V, device="cuda", generator=gen) * 2.0).to(torch.bfloat16)
    w = torch.linspace(0.5, 1.5, V, device="cuda")
    o, ht = kairos_gdn.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=h0,
                                              output_final_state=True)
    monkeypatch.setenv("KAIROS_GDN_FUSED_NORM", "1")
    y, ht2 = kairos_gdn.chunk_gated_delta_rule_gated_norm(d["q"], d["k"], d["v"], d["g"], d["beta"], gate, w,
                                                          initial_state=h0, output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(ht2, ht)
    sel = slice(0, T, 97)
    o_s = o[:, sel].float().cpu().numpy().reshape(-1, V)
    g_s = gate[:, sel].float().cpu().numpy().reshape(-1, V).astype(np.float64)
    y_ref, _ = O.rms_norm_gated(o_s, g_s, w.cpu().numpy().astype(np.float64), None, "swish", 1e-5, dtype="bf16")
    _within_ulp(y[:, sel].reshape(-1, V), y_ref, "bf16")
    # every token: the fused call against the plain forward followed by the norm kernel
    y_sep = kairos_gdn.rms_norm_gated_fwd(o.reshape(-1, V), gate.reshape(-1, V), w, None, "swish", 1e-5)
    diff = (y.reshape(-1, V).float() - y_sep.float()).abs()
    ulp = y_sep.float().abs().clamp_min(1e-30) * 2.0 ** -7
    assert bool((diff <= ulp).all())
    assert float((diff == 0).float().mean()) >= 0.99


@pytest.mark.parametrize("form", ["parts", "fold"])
@pytest.mark.parametrize("l2", [True, False])
def test_gated_norm_model_shape_full_size(l2, form, monkeypatch):
    """The Kairos layer (T=32760, H=20, dk=256, dv=512, bf16, in-op L2 norm as the layer calls it),
    against the plain forward followed by the norm kernel on every token, and against the oracle's
    norm of the plain forward's o on every 97th token.  "parts" (the default): the norm kernel on each
    pipelined part's rows beside the next part's recurrence, bit-identical to the two-step form (every
    row normalised exactly once); "fold": the norm in the fused K = 256 kernel
    (KAIROS_GDN_WIDE_NORM_FOLD=1), within one bf16 ulp and >= 99% identical."""
    B, T, H, K, V = 1, 32760, 20, 256, 512
    note(f"chunk_fwd_gated_norm full size B={B} T={T} H={H} K={K} V={V} l2={l2} form={form}")
    gen = torch.Generator(device="cuda").manual_seed(11)
    r = lambda *sh: torch.randn(*sh, device="cuda", generator=gen)  # noqa: E731
    q = r(B, T, H, K)
    k = r(B, T, H, K)
    if not l2:
        q = q / q.norm(dim=-1, keepdim=True)
        k = k / k.norm(dim=-1, keepdim=True)
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    v = r(B, T, H, V).to(torch.bfloat16)
    beta = torch.sigmoid(r(B, T, H)).to(torch.bfloat16)
    g = -torch.nn.functional.softplus(r(B, T, H))
    h0 = 0.02 * r(B, H, K, V)
    gate = (r(B, T, H, V) * 2.0).to(torch.bfloat16)
    w = torch.linspace(0.5, 1.5, V, device="cuda")
    bias = torch.linspace(-0.1, 0.1, V, device="cuda")
    o, ht = kairos_gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                                              use_qk_l2norm_in_kernel=l2)
    monkeypatch.setenv("KAIROS_GDN_FUSED_NORM", "1")
    monkeypatch.setenv("KAIROS_GDN_NORM_PARTS", "1")
    monkeypatch.setenv("KAIROS_GDN_WIDE_NORM_FOLD", "1" if form == "fold" else "0")
    y, ht2 = kairos_gdn.chunk_gated_delta_rule_gated_norm(q, k, v, g, beta, gate, w, bias, initial_state=h0,
                                                          output_final_state=True, use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    assert torch.equal(ht2, ht)
    assert bool(torch.isfinite(y).all())
    y_sep = kairos_gdn.rms_norm_gated_fwd(o.reshape(-1, V), gate.reshape(-1, V), w, bias, "swish", 1e-5)
    if form == "parts":
        assert torch.equal(y.reshape(-1, V), y_sep)
    diff = (y.reshape(-1, V).float() - y_sep.float()).abs()
    mag = (o.reshape(-1, V).float().abs() * w.abs() + bias.abs()) * gate.reshape(-1, V).float().abs()
    ulp = y_sep.float().abs().clamp_min(1e-30) * 2.0 ** -7 + mag * 2.0 ** -20
    assert bool((diff <= ulp).all()), float((diff - ulp).max())
    same = float((diff == 0).float().mean())
    note(f"    identical to the two-step form: {same:.4f}")
    assert same >= 0.99
    sel = slice(0, T, 97)
    o_s = o[:, sel].float().cpu().numpy().reshape(-1, V)
    g_s = gate[:, sel].float().cpu().numpy().reshape(-1, V).astype(np.float64)
    y_ref, _ = O.rms_norm_gated(o_s, g_s, w.cpu().numpy().astype(np.float64), bias.cpu().numpy().astype(np.float64),
                                "swish", 1e-5, dtype="bf16")
    mag_s = _magnitude(o_s, g_s, w.cpu().numpy().astype(np.float64), bias.cpu().numpy().astype(np.float64),
                       "swish", 1e-5)
    _within_ulp(y[:, sel].reshape(-1, V), y_ref, "bf16", mag_s)


@pytest.mark.parametrize("parts,growth", [("2", "1.4"), ("5", "1"), ("10", "1.4")])
def test_gated_norm_by_parts_pipeline_shapes(parts, growth, monkeypatch):
    """The norm by parts over other pipeline cuts of the K = 256 forward (two parts; five equal parts;
    ten parts) on two sequences: bit-identical to the forward followed by the
    norm kernel over all rows (every row normalised exactly once).  T = 1300: 21 chunks, so ten
    parts (the most a sequence of 21 chunks is cut into) hold two or three chunks each."""
    B, T, H, K, V = 2, 1300, 2, 256, 128
    note(f"gated norm by parts: parts={parts} growth={growth} B={B} T={T} H={H} K={K} V={V}")
    monkeypatch.setenv("KAIROS_GDN_WIDE_PIPE", parts)
    monkeypatch.setenv("KAIROS_GDN_WIDE_PIPE_GROWTH", growth)
    monkeypatch.setenv("KAIROS_GDN_WIDE_NORM_FOLD", "0")
    gen = torch.Generator(device="cuda").manual_seed(int(parts) + 17)
    r = lambda *sh: torch.randn(*sh, device="cuda", generator=gen)  # noqa: E731
    q = r(B, T, H, K).to(torch.bfloat16)
    k = r(B, T, H, K).to(torch.bfloat16)
    v = r(B, T, H, V).to(torch.bfloat16)
    beta = torch.sigmoid(r(B, T, H)).to(torch.bfloat16)
    g = -torch.nn.functional.softplus(r(B, T, H))
    h0 = 0.02 * r(B, H, K, V)
    gate = (r(B, T, H, V) * 2.0).to(torch.bfloat16)
    w = torch.linspace(0.5, 1.5, V, device="cuda")
    o, ht = kairos_gdn.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=h0, output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
    y_ref = kairos_gdn.rms_norm_gated_fwd(o.reshape(-1, V), gate.reshape(-1, V), w, None, "swish", 1e-5)
    for mode in ("1", "0"):
        monkeypatch.setenv("KAIROS_GDN_NORM_PARTS", mode)
        y, ht2 = kairos_gdn.chunk_gated_delta_rule_gated_norm(q, k, v, g, beta, gate, w, initial_state=h0,
                                                              output_final_state=True, use_qk_l2norm_in_kernel=True)
        torch.cuda.synchronize()
        assert torch.equal(ht2, ht)
        assert torch.equal(y.reshape(-1, V), y_ref), f"norm parts={mode}"


def test_gated_norm_argument_errors():
    x = make_inputs(1, 64, 1, 64, 64, seed=1, dtype="bf16")
    d = {k: dev(x[k], torch.bfloat16) for k in ("q", "k", "v", "beta")}
    d["g"] = dev(x["g"])
    gate = torch.zeros(1, 64, 1, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="Unsupported activation"):
        kairos_gdn.chunk_gated_delta_rule_gated_norm(d["q"], d["k"], d["v"], d["g"], d["beta"], gate,
                                                     activation="relu")
    with pytest.raises(ValueError, match="gate shape"):
        kairos_gdn.chunk_gated_delta_rule_gated_norm(d["q"], d["k"], d["v"], d["g"], d["beta"], gate[:, :32])
    with pytest.raises(ValueError, match="norm_weight must have shape"):
        kairos_gdn.chunk_gated_delta_rule_gated_norm(d["q"], d["k"], d["v"], d["g"], d["beta"], gate,
                                                     torch.ones(32, device="cuda"))
