"""GPU parity of the HIP kernels against the CPU oracle, through the C ABI.

Tolerances (relative L2 = RMS(err) / RMS(ref), fla's get_err_ratio):
  bf16 path: o <= 1e-2, final_state <= 5e-3;
             stage intermediates (w, u, h, v_new) <= 1e-2, fp32 gc / A <= 1e-5.
  fp32 path: o, final_state and every intermediate <= 1e-4.
Full-size configs compare every head on the GPU against the oracle on a
subset of heads (heads are independent), plus size-independent properties:
determinism, varlen == separate calls, split calls with state carry.
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
from gdn_inputs import CONFIGS, dequant_bf16, make_inputs, quantize_fp8
import kairos_gdn

pytestmark = pytest.mark.gpu

TOL = {"bf16": dict(o=1e-2, ht=5e-3, mid=1e-2), "fp32": dict(o=1e-4, ht=1e-4, mid=1e-4)}
TDT = {"bf16": torch.bfloat16, "fp32": torch.float32}


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dev(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda").to(dtype)


def host(t):
    return t.detach().float().cpu().numpy()


def to_dev(x, dt):
    d = {k: dev(x[k], TDT[dt]) for k in ("q", "k", "v")}
    d["beta"] = dev(x["beta"], TDT[dt])
    d["g"] = dev(x["g"], torch.float32)
    d["h0"] = dev(x["h0"]) if x["h0"] is not None else None
    return d


def chunk_T_to_tokens(xT, cm, rows=64):
    """[NCb, H, V, 64] per-chunk transposed -> [B, T, H, V] (oracle ChunkMap order)."""
    a = np.swapaxes(xT[:cm.nc], 2, 3)                    # [NC, H, 64, V]
    return cm.scatter(a, np.float32)


def tokens_to_chunk_T(x, cm, ncb):
    """[B, T, H, V] -> [NCb, H, V, 64] (zeros in padded rows and spare chunks)."""
    a = np.swapaxes(cm.gather(x, np.float32), 2, 3)       # [NC, H, V, 64]
    out = np.zeros((ncb,) + a.shape[1:], np.float32)
    out[:cm.nc] = a
    return out


def rel(a, b):
    return O.rel_l2(a, b)


@pytest.fixture(scope="module", autouse=True)
def _gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    kairos_gdn._lib.load()


# ---------------------------------------------------------------------------
# elementwise stages
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["bf16", "fp32"])
def test_l2norm(dt):
    note(f"l2norm {dt}")
    rng = np.random.default_rng(0)
    x = O.cast(rng.standard_normal((3, 777, 128)).astype(np.float32) * 3, dt)
    y, rstd = kairos_gdn.l2norm_fwd(dev(x, TDT[dt]))
    ref = O.l2norm(x, dtype=dt)
    assert rel(host(y), ref) < (4e-3 if dt == "bf16" else 1e-6)
    assert tuple(rstd.shape) == x.shape[:-1] and rstd.dtype == torch.float32
    rs_ref = 1.0 / np.sqrt((x.astype(np.float64) ** 2).sum(-1) + 1e-6)
    assert rel(host(rstd), rs_ref) < 1e-6


@pytest.mark.parametrize("cu", [None, [0, 1, 64, 65, 200, 330]])
def test_cumsum(cu):
    note(f"cumsum cu={cu}")
    rng = np.random.default_rng(1)
    B = 1 if cu else 2
    g = (-np.logaddexp(0, rng.standard_normal((B, 330, 5)))).astype(np.float32)
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    gc = host(kairos_gdn.chunk_local_cumsum(dev(g), cu_seqlens=cu_t))
    ref = O.chunk_local_cumsum(g, cu_seqlens=np.array(cu) if cu else None)
    np.testing.assert_allclose(gc, ref, rtol=1e-5, atol=2e-5)


# ---------------------------------------------------------------------------
# prepare (cumsum + K.K^T + solve + w/u), fed identical inputs
# ---------------------------------------------------------------------------
PREP_CASES = [
    ("bf16", 1, 300, 3, 128, 128, None),
    ("bf16", 2, 200, 2, 64, 128, None),
    ("bf16", 1, 400, 2, 128, 64, [0, 10, 74, 74, 260, 400]),
    ("fp32", 1, 200, 2, 64, 64, None),
    ("fp32", 1, 150, 2, 128, 128, [0, 100, 150]),
    # Kairos model head dims (K = 256, V = 512): v staged in two 256-column passes
    ("bf16", 1, 200, 2, 256, 512, None),
    # fp32 K = 256 at the LDS limit: 128-column passes
    ("fp32", 1, 130, 1, 256, 256, None),
    # V = 320: a ragged last pass of 64 columns
    ("bf16", 1, 150, 2, 128, 320, [0, 70, 150]),
]


@pytest.mark.parametrize("dt,B,T,H,K,V,cu", PREP_CASES)
def test_prepare_stage(dt, B, T, H, K, V, cu):
    note(f"prepare {dt} B={B} T={T} H={H} K={K} V={V} cu={cu}")
    x = make_inputs(B, T, H, K, V, seed=T + K + V, dtype=dt, n_states=len(cu) - 1 if cu else None)
    d = to_dev(x, dt)
    cu_np = np.array(cu) if cu else None
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    gc, w, uT, A, Ai = kairos_gdn.prepare_wy(d["k"], d["v"], d["g"], d["beta"], cu_seqlens=cu_t, return_A=True)
    torch.cuda.synchronize()
    cm = O.ChunkMap(B, T, cu_np)
    gc_r = O.chunk_local_cumsum(x["g"], cu_np, dtype=dt)
    np.testing.assert_allclose(host(gc), gc_r, rtol=1e-5, atol=2e-5)
    A_r = O.chunk_scaled_dot_kkt(x["k"], gc_r, x["beta"], cu_np, dtype=dt)
    assert rel(host(A), A_r) < 1e-5
    Ai_r = O.solve_tril(A_r, cu_np, dtype=dt)
    assert rel(host(Ai), Ai_r) < TOL[dt]["mid"] / 2
    w_r, u_r = O.recompute_w_u(x["k"], x["v"], x["beta"], Ai_r, gc_r, cu_np, dtype=dt)
    assert rel(host(w), w_r) < TOL[dt]["mid"]
    assert rel(chunk_T_to_tokens(host(uT), cm), u_r) < TOL[dt]["mid"]
    # padded rows of the transposed u are exact zeros (the later stages rely on it)
    ut = host(uT)[:cm.nc]
    pad = ~cm.valid
    assert np.all(np.swapaxes(ut, 2, 3)[pad[:, None, :].repeat(H, 1)] == 0)


# ---------------------------------------------------------------------------
# state recurrence and output, fed the oracle's own intermediates
# ---------------------------------------------------------------------------
H_CASES = [
    ("bf16", 1, 520, 3, 128, 128, None, True),
    ("bf16", 2, 130, 2, 64, 64, None, False),
    ("bf16", 1, 500, 2, 128, 128, [0, 63, 64, 64, 300, 500], True),
    ("fp32", 1, 260, 2, 64, 64, None, True),
    ("bf16", 1, 300, 2, 256, 512, None, True),
    ("fp32", 1, 150, 1, 256, 128, [0, 20, 150], True),
]


@pytest.mark.parametrize("dt,B,T,H,K,V,cu,with_h0", H_CASES)
def test_fwd_h_and_fwd_o_stages(dt, B, T, H, K, V, cu, with_h0):
    note(f"fwd_h/fwd_o {dt} B={B} T={T} H={H} K={K} V={V} cu={cu} h0={with_h0}")
    x = make_inputs(B, T, H, K, V, seed=7 * T + K, dtype=dt, n_states=len(cu) - 1 if cu else None,
                    h0_scale=0.02 if with_h0 else 0.0)
    cu_np = np.array(cu) if cu else None
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    o_r, ht_r, inter = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                                output_final_state=True, cu_seqlens=cu_np, dtype=dt,
                                                return_intermediates=True)
    cm = O.ChunkMap(B, T, cu_np)
    ncb = kairos_gdn.num_chunks_bound(B, T, len(cu) - 1 if cu else 0)
    d = to_dev(x, dt)
    w = dev(inter["w"], TDT[dt])
    uT = dev(tokens_to_chunk_T(inter["u"], cm, ncb), TDT[dt])
    gc = dev(inter["gc"])
    hT, vnT, ht = kairos_gdn.fwd_h(d["k"], w, uT, gc, initial_state=d["h0"], output_final_state=True,
                                   cu_seqlens=cu_t)
    torch.cuda.synchronize()
    h_gpu = np.swapaxes(host(hT)[:cm.nc], 2, 3)
    assert rel(h_gpu, inter["h"]) < TOL[dt]["mid"]
    assert rel(chunk_T_to_tokens(host(vnT), cm), inter["v_new"]) < TOL[dt]["mid"]
    assert rel(host(ht), ht_r) < TOL[dt]["ht"]
    # output stage on the oracle's h and v_new
    hT_r = np.zeros((ncb, H, V, K), np.float32)
    hT_r[:cm.nc] = np.swapaxes(inter["h"], 2, 3)
    o = kairos_gdn.fwd_o(d["q"], d["k"], dev(hT_r, TDT[dt]), dev(tokens_to_chunk_T(inter["v_new"], cm, ncb), TDT[dt]),
                         gc, cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert rel(host(o), o_r) < TOL[dt]["o"]


@pytest.mark.parametrize("dt,B,T,H,K,V,cu,with_h0", H_CASES)
def test_reference_layout_stages(dt, B, T, H, K, V, cu, with_h0):
    """recompute_w_u_fwd / chunk_gated_delta_rule_fwd_h / chunk_fwd_o in the reference's layouts:
    u, v_new [B,T,H,V] and h [NT,H,K,V] compared with the oracle's intermediates as they are,
    with no layout helper of the tests in between; h's slack chunks are zeros and the layout
    moves are exact (the tokens form equals the tiled form bit for bit)."""
    note(f"reference-layout stages {dt} B={B} T={T} H={H} K={K} V={V} cu={cu} h0={with_h0}")
    x = make_inputs(B, T, H, K, V, seed=11 * T + K, dtype=dt, n_states=len(cu) - 1 if cu else None,
                    h0_scale=0.02 if with_h0 else 0.0)
    cu_np = np.array(cu) if cu else None
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    o_r, ht_r, inter = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                                output_final_state=True, cu_seqlens=cu_np, dtype=dt,
                                                return_intermediates=True)
    cm = O.ChunkMap(B, T, cu_np)
    d = to_dev(x, dt)
    gc, w, u = kairos_gdn.recompute_w_u_fwd(d["k"], d["v"], d["beta"], g_raw=d["g"], cu_seqlens=cu_t)
    _, w2, uT, _, _ = kairos_gdn.prepare_wy(d["k"], d["v"], d["g"], d["beta"], cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert torch.equal(w, w2)
    ncb = kairos_gdn.num_chunks_bound(B, T, len(cu) - 1 if cu else 0)
    assert np.array_equal(host(u), chunk_T_to_tokens(host(uT), cm))
    assert rel(host(u), inter["u"]) < TOL[dt]["mid"]
    # the recurrence fed the oracle's own w, u (reference layouts)
    gc_r = dev(inter["gc"])
    h, v_new, ht = kairos_gdn.chunk_gated_delta_rule_fwd_h(d["k"], dev(inter["w"], TDT[dt]), dev(inter["u"], TDT[dt]),
                                                           gc_r, initial_state=d["h0"], output_final_state=True,
                                                           cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert tuple(h.shape) == (ncb, H, K, V)
    assert rel(host(h)[:cm.nc], inter["h"]) < TOL[dt]["mid"]
    assert np.all(host(h)[cm.nc:] == 0)
    assert rel(host(v_new), inter["v_new"]) < TOL[dt]["mid"]
    assert rel(host(ht), ht_r) < TOL[dt]["ht"]
    hT, vnT, _ = kairos_gdn.fwd_h(d["k"], dev(inter["w"], TDT[dt]),
                                  dev(tokens_to_chunk_T(inter["u"], cm, ncb), TDT[dt]), gc_r,
                                  initial_state=d["h0"], cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert np.array_equal(host(h)[:cm.nc], np.swapaxes(host(hT)[:cm.nc], 2, 3))
    assert np.array_equal(host(v_new), chunk_T_to_tokens(host(vnT), cm))
    # the output stage fed the oracle's own h and v_new (reference layouts)
    h_r = np.zeros((ncb, H, K, V), np.float32)
    h_r[:cm.nc] = inter["h"]
    o = kairos_gdn.chunk_fwd_o(d["q"], d["k"], dev(inter["v_new"], TDT[dt]), dev(h_r, TDT[dt]), gc_r,
                               cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert rel(host(o), o_r) < TOL[dt]["o"]


@pytest.mark.parametrize("dt,B,T,H,K,V,cu,with_h0", [c for c in H_CASES if c[0] == "bf16" and c[4] <= 128])
def test_fwd_h_split_k_form(dt, B, T, H, K, V, cu, with_h0, monkeypatch):
    """bf16 K, V <= 128 run the all-columns recurrence; KAIROS_GDN_FWD_H_COLS=0 selects the split-K form,
    checked here on the same cases."""
    monkeypatch.setenv("KAIROS_GDN_FWD_H_COLS", "0")
    test_fwd_h_and_fwd_o_stages(dt, B, T, H, K, V, cu, with_h0)


# ---------------------------------------------------------------------------
# whole op
# ---------------------------------------------------------------------------
def run_gpu(x, dt, cu=None, l2=False, out_final=True, with_h0=True):
    d = to_dev(x, dt)
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu is not None else None
    o, ht = kairos_gdn.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"],
                                              initial_state=d["h0"] if with_h0 else None,
                                              output_final_state=out_final, cu_seqlens=cu_t,
                                              use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    return o, ht


def check_against_oracle(x, dt, o, ht, cu=None, heads=None, l2=False, with_h0=True):
    sel = slice(None) if heads is None else np.array(heads)
    xs = {k: (v[:, :, sel] if k != "h0" else (v[:, sel] if v is not None else None)) for k, v in x.items()}
    o_r, ht_r = O.chunk_gated_delta_rule(xs["q"], xs["k"], xs["v"], xs["g"], xs["beta"],
                                         initial_state=xs["h0"] if with_h0 else None, output_final_state=True,
                                         cu_seqlens=np.array(cu) if cu is not None else None,
                                         use_qk_l2norm_in_kernel=l2, dtype=dt)
    eo = rel(host(o)[:, :, sel], o_r)
    eh = rel(host(ht)[:, sel], ht_r) if ht is not None else 0.0
    note(f"    rel-L2 o={eo:.3e} ht={eh:.3e}")
    assert eo < TOL[dt]["o"]
    assert eh < TOL[dt]["ht"]
    return eo, eh


EDGE_CASES = [
    # dt, B, T, H, K, V, cu, l2, with_h0
    ("bf16", 1, 1, 2, 64, 64, None, False, True),
    ("bf16", 1, 63, 2, 128, 128, None, False, True),
    ("bf16", 3, 200, 2, 128, 64, None, False, True),
    ("bf16", 1, 1000, 4, 128, 128, None, True, True),
    ("bf16", 1, 700, 3, 64, 128, [0, 1, 1, 129, 640, 700], False, True),
    ("bf16", 2, 100, 2, 64, 64, None, False, False),
    ("fp32", 2, 300, 2, 128, 128, None, False, True),
    # the Kairos 4B layer's head dims and its in-kernel L2 norm (GatedDeltaNet defaults
    # head_dim=256, expand_v=2: layers/gated_deltanet.py:90-93,122-123)
    ("bf16", 1, 300, 2, 256, 512, None, True, True),
    ("bf16", 1, 400, 2, 256, 512, [0, 1, 130, 400], False, True),
    # a last chunk of 20 tokens: gate shuffles in ragged chunks must read from active lanes
    ("bf16", 1, 1300, 2, 256, 512, None, False, True),
    ("fp32", 1, 200, 1, 256, 256, None, False, True),
    # the fused K = 256 kernel with 3 and 1 value tiles per head (its L2 prefetch splits rows over
    # the tiles), two batch rows with a ragged end, and varlen cuts at chunk edges
    ("bf16", 2, 260, 3, 256, 192, None, False, True),
    ("bf16", 1, 500, 2, 256, 64, [0, 63, 64, 65, 500], True, True),
    ("bf16", 2, 150, 2, 128, 48, None, False, True),
    # the in-op L2 norm on the fused path at K = 64 (8 lanes per row) with ragged varlen chunks
    ("bf16", 1, 700, 3, 64, 128, [0, 1, 1, 129, 640, 700], True, True),
    ("bf16", 2, 333, 2, 128, 64, None, True, False),
]


@pytest.mark.parametrize("dt,B,T,H,K,V,cu,l2,with_h0", EDGE_CASES)
def test_full_op_edge_cases(dt, B, T, H, K, V, cu, l2, with_h0):
    note(f"chunk_gated_delta_rule {dt} B={B} T={T} H={H} K={K} V={V} cu={cu} l2={l2} h0={with_h0}")
    n = len(cu) - 1 if cu else None
    x = make_inputs(B, T, H, K, V, seed=T * 3 + H, dtype=dt, n_states=n, h0_scale=0.02 if with_h0 else 0.0)
    if l2:                                   # un-normalised q/k: the kernel normalises them
        x["q"] = O.cast(x["q"] * 3.0, dt)
        x["k"] = O.cast(x["k"] * 0.5, dt)
    o, ht = run_gpu(x, dt, cu=cu, l2=l2, with_h0=with_h0)
    assert o.dtype == TDT[dt] and tuple(o.shape) == (B, T, H, V)
    assert ht.dtype == torch.float32
    check_against_oracle(x, dt, o, ht, cu=cu, l2=l2, with_h0=with_h0)


@pytest.mark.parametrize("cu", [None, [0, 1, 130, 400]])
def test_model_head_dims_stage_kernels(cu, monkeypatch):
    """K=256, V=512 through the stage kernels (fwd_h + fwd_o, KAIROS_GDN_WIDE_FUSED=0) instead of the
    fused recurrence + output: both forms against the oracle."""
    monkeypatch.setenv("KAIROS_GDN_WIDE_FUSED", "0")
    note(f"stage kernels K=256 V=512 cu={cu}")
    n = len(cu) - 1 if cu else None
    x = make_inputs(1, 400, 2, 256, 512, seed=41, dtype="bf16", n_states=n)
    o, ht = run_gpu(x, "bf16", cu=cu)
    check_against_oracle(x, "bf16", o, ht, cu=cu)


@pytest.mark.parametrize("with_h0", [True, False])
def test_model_head_dims_pipeline_parts(with_h0, monkeypatch):
    """The K=256 forward cut into P parts along each sequence (prepare of the next part on a second
    stream beside the recurrence of this one, the state carried in fp32 between parts) gives the
    same bits as one part: two sequences, a ragged last chunk, 13 chunks in 2, 3, 4 and 6 equal parts
    and in parts that grow or shrink along the sequence."""
    note(f"K=256 pipeline parts h0={with_h0}")
    x = make_inputs(2, 64 * 12 + 37, 2, 256, 128, seed=43, dtype="bf16", h0_scale=0.02 if with_h0 else 0.0)
    monkeypatch.setenv("KAIROS_GDN_WIDE_PIPE", "1")
    o1, ht1 = run_gpu(x, "bf16", with_h0=with_h0)
    check_against_oracle(x, "bf16", o1, ht1, with_h0=with_h0)
    for parts, growth in (("2", "1"), ("3", "1"), ("4", "1"), ("6", "1"), ("4", "1.3"), ("3", "2.5"), ("6", "0.7")):
        monkeypatch.setenv("KAIROS_GDN_WIDE_PIPE", parts)
        monkeypatch.setenv("KAIROS_GDN_WIDE_PIPE_GROWTH", growth)
        o, ht = run_gpu(x, "bf16", with_h0=with_h0)
        assert torch.equal(o, o1), (parts, growth)
        assert torch.equal(ht, ht1), (parts, growth)


def test_empty_sequence_returns_initial_state():
    note("T=0")
    x = make_inputs(2, 0, 2, 64, 64, seed=1, dtype="bf16")
    o, ht = run_gpu(x, "bf16")
    assert o.numel() == 0
    np.testing.assert_array_equal(host(ht), x["h0"])


def test_bf16_gates_and_state_inputs():
    note("bf16 g / beta / h0")
    x = make_inputs(1, 300, 2, 128, 128, seed=5, dtype="bf16")
    x["g"] = O.to_bf16(x["g"])
    d = to_dev(x, "bf16")
    o, ht = kairos_gdn.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"].bfloat16(), d["beta"],
                                              initial_state=d["h0"].bfloat16(), output_final_state=True)
    torch.cuda.synchronize()
    x["h0"] = O.to_bf16(x["h0"])
    check_against_oracle(x, "bf16", o, ht)


@pytest.mark.parametrize("K,V,cu,l2", [(128, 128, None, False), (64, 128, [0, 1, 130, 300], True),
                                      (256, 512, None, True)])
def test_fp16_inputs(K, V, cu, l2):
    """fp16 q/k/v/beta (the reference op is dtype-generic): computed by the fp32 kernels, o in fp16.
    Against the fp32-cast-point oracle on the same fp16 values: o within its own fp16 rounding
    (<= 2e-3), final_state <= 1e-4; against the fp64 token recurrence within the north-star bar."""
    note(f"fp16 inputs K={K} V={V} cu={cu} l2={l2}")
    T = 300
    x = make_inputs(1, T, 2, K, V, seed=11, dtype="fp32", n_states=len(cu) - 1 if cu else 1)
    f16 = lambda a: a.astype(np.float16).astype(np.float32)  # noqa: E731
    for n in ("q", "k", "v", "beta"):
        x[n] = f16(x[n] * (1.7 if (l2 and n in ("q", "k")) else 1.0))
    d = {n: dev(x[n], torch.float16) for n in ("q", "k", "v", "beta")}
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    o, ht = kairos_gdn.chunk_gated_delta_rule(d["q"], d["k"], d["v"], dev(x["g"]), d["beta"],
                                              initial_state=dev(x["h0"]), output_final_state=True,
                                              use_qk_l2norm_in_kernel=l2, cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert o.dtype == torch.float16 and ht.dtype == torch.float32
    o_r, ht_r = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                         output_final_state=True, use_qk_l2norm_in_kernel=l2,
                                         cu_seqlens=np.array(cu) if cu else None, dtype="fp32")
    eo, eh = rel(host(o), o_r), rel(host(ht), ht_r)
    nrm = (lambda a: a / np.sqrt(np.sum(np.square(a.astype(np.float64)), -1, keepdims=True) + 1e-6)) if l2 \
        else (lambda a: a)
    o_n, ht_n = O.naive_recurrent(nrm(x["q"]), nrm(x["k"]), x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                  cu_seqlens=np.array(cu) if cu else None)
    en, ehn = rel(host(o), o_n), rel(host(ht), ht_n)
    note(f"    rel-L2 vs fp32 oracle: o={eo:.3e} ht={eh:.3e}; vs fp64 recurrence: o={en:.3e} ht={ehn:.3e}")
    assert eo < 2e-3 and eh < 1e-4
    assert en < 1e-2 and ehn < 5e-3


@pytest.mark.parametrize("cfg", [0, 1])
def test_baseline_config(cfg):
    c = CONFIGS[cfg]
    note(f"config {cfg}: {c}")
    x = make_inputs(c["B"], c["T"], c["H"], c["K"], c["V"], seed=20260 + cfg, dtype=c["dtype"],
                    h0_scale=0.0 if c.get("zero_h0") else 0.02)
    if c.get("zero_h0"):
        x["h0"] = np.zeros((c["B"], c["H"], c["K"], c["V"]), np.float32)
    o, ht = run_gpu(x, c["dtype"])
    check_against_oracle(x, c["dtype"], o, ht)
    if cfg == 0:                             # config 0 also checks against the fp64 token recurrence
        on, hn = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"])
        assert rel(host(o), on) < 1e-4 and rel(host(ht), hn) < 1e-4


@pytest.mark.parametrize("cfg,l2", [(2, False), (3, False), (2, True)])
def test_baseline_config_full_size(cfg, l2):
    """Configs 2 and 3 at full size, every head against the oracle; config 2 also in the layer's own mode,
    use_qk_l2norm_in_kernel=True on unnormalised q, k."""
    c = CONFIGS[cfg]
    note(f"config {cfg}, all heads, l2={l2}")
    cu = c.get("cu")
    x = make_inputs(c["B"], c["T"], c["H"], c["K"], c["V"], seed=20260 + cfg, dtype=c["dtype"],
                    n_states=len(cu) - 1 if cu else None)
    if l2:
        x["q"] = O.cast(x["q"] * 3.0, c["dtype"])
        x["k"] = O.cast(x["k"] * 0.5, c["dtype"])
    o, ht = run_gpu(x, c["dtype"], cu=cu, l2=l2)
    assert bool(torch.isfinite(o).all()) and bool(torch.isfinite(ht).all())
    check_against_oracle(x, c["dtype"], o, ht, cu=cu, l2=l2)


def test_varlen_maps_bit_exact():
    """The device-built varlen maps: chunk offsets == prepare_chunk_offsets(cu_seqlens, 64)
    (index.py:122-127) and segment offsets == the cumulative ceil(chunks / L), bit for bit, with empty
    and 1-token sequences and lengths at chunk boundaries."""
    lib = kairos_gdn._lib.load()
    rng = np.random.default_rng(7)
    lens = [0, 1, 63, 64, 65, 0, 128, 129, 1, 0, 4095, 4096, 4097, 640, 7]
    lens += [int(x) for x in rng.integers(0, 3000, 40)]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    N = len(lens)
    nch = (np.array(lens) + 63) // 64
    for L in (1, 3, 43, 100000):
        cu_t = torch.from_numpy(cu).to("cuda")
        co = torch.full((N + 1,), -1, dtype=torch.int32, device="cuda")
        so = torch.full((N + 1,), -1, dtype=torch.int32, device="cuda")
        kairos_gdn._lib.check("kairos_gdn_varlen_maps",
                              lib.kairos_gdn_varlen_maps(cu_t.data_ptr(), N, L, co.data_ptr(), so.data_ptr(),
                                                         torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(co.cpu().numpy(), np.concatenate([[0], np.cumsum(nch)]))
        np.testing.assert_array_equal(so.cpu().numpy(), np.concatenate([[0], np.cumsum((nch + L - 1) // L)]))


@pytest.mark.parametrize("l2", [False, True], ids=["plain", "l2norm"])
def test_model_shape_full_size(l2):
    """The Kairos 4B layer at the headline clip length: H=20, K=256, V=512, T=32760, bf16, against the
    oracle on every head (child processes over head groups, tests/oracle_pool.py).  With l2, the
    layer's own mode: unnormalised q, k and use_qk_l2norm_in_kernel=True (gated_deltanet.py:275-285),
    which the fused K = 256 path folds into prepare and the recurrence."""
    import oracle_pool
    B, T, H, K, V = 1, 32760, 20, 256, 512
    note(f"model shape B={B} T={T} H={H} K={K} V={V} l2={l2} (oracle on all {H} heads)")
    x = make_inputs(B, T, H, K, V, seed=20270, dtype="bf16")
    if l2:
        rng = np.random.default_rng(20271)
        for n in ("q", "k"):
            x[n] = O.to_bf16(x[n] * rng.uniform(0.5, 3.0, x[n].shape[:-1] + (1,)).astype(np.float32))
    o, ht = run_gpu(x, "bf16", l2=l2)
    assert bool(torch.isfinite(o).all()) and bool(torch.isfinite(ht).all())
    note("    HIP forward done; oracle on every head")
    e = oracle_pool.forward_all_heads(x, host(o), host(ht), "bf16", workers=8, group=2, log=note,
                                      use_qk_l2norm_in_kernel=l2)
    note(f"    rel-L2 over all heads o={e['o']:.3e} ht={e['ht']:.3e}")
    assert e["o"] < TOL["bf16"]["o"] and e["ht"] < TOL["bf16"]["ht"]


# ---------------------------------------------------------------------------
# size-independent properties at the full sizes
# ---------------------------------------------------------------------------
def test_full_size_properties():
    c = CONFIGS[3]
    cu = c["cu"]
    note("properties: determinism, varlen == separate calls, split with state carry")
    x = make_inputs(1, c["T"], c["H"], c["K"], c["V"], seed=99, dtype="bf16", n_states=len(cu) - 1)
    d = to_dev(x, "bf16")
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda")
    f = kairos_gdn.chunk_gated_delta_rule
    o1, h1 = f(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"], output_final_state=True,
               cu_seqlens=cu_t)
    o2, h2 = f(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"], output_final_state=True,
               cu_seqlens=cu_t)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(h1, h2)                  # deterministic
    # varlen == separate calls.  The two calls cut the sequences into different
    # segments, whose initial states come from the fp32 segment scan instead of
    # the bf16-snapshot recurrence, so they agree to rounding, not bitwise.
    for n in range(len(cu) - 1):
        s = slice(cu[n], cu[n + 1])
        on, hn = f(d["q"][:, s], d["k"][:, s], d["v"][:, s], d["g"][:, s], d["beta"][:, s],
                   initial_state=d["h0"][n:n + 1], output_final_state=True)
        torch.cuda.synchronize()
        eo, eh = rel(host(on), host(o1[:, s])), rel(host(hn), host(h1[n:n + 1]))
        note(f"    seq {n}: varlen vs separate rel-L2 o={eo:.2e} ht={eh:.2e}")
        assert eo < 2e-3 and eh < 2e-3
    # the last sequence split at a chunk boundary with the state carried
    s0, s1 = cu[3], cu[4]
    mid = s0 + 64 * 200
    oa, ha = f(d["q"][:, s0:mid], d["k"][:, s0:mid], d["v"][:, s0:mid], d["g"][:, s0:mid], d["beta"][:, s0:mid],
               initial_state=d["h0"][3:4], output_final_state=True)
    ob, hb = f(d["q"][:, mid:s1], d["k"][:, mid:s1], d["v"][:, mid:s1], d["g"][:, mid:s1], d["beta"][:, mid:s1],
               initial_state=ha, output_final_state=True)
    torch.cuda.synchronize()
    eo = rel(host(torch.cat([oa, ob], 1)), host(o1[:, s0:s1]))
    eh = rel(host(hb), host(h1[3:4]))
    note(f"    split with state carry vs one call rel-L2 o={eo:.2e} ht={eh:.2e}")
    assert eo < 2e-3 and eh < 2e-3


# ---------------------------------------------------------------------------
# segment scan: slow gates make the per-segment transition [M | R] and the
# fp32 combine carry real signal across many chunks
# ---------------------------------------------------------------------------
def slow_gate_inputs(B, T, H, K, V, seed, n_states=None):
    x = make_inputs(B, T, H, K, V, seed=seed, dtype="bf16", n_states=n_states, h0_scale=0.5)
    x["g"] = (x["g"] * 0.004).astype(np.float32)       # ~ -0.003 per token: decay e^-0.2 per chunk
    return x


@pytest.mark.parametrize("L", ["1", "3", "8", "64"])
@pytest.mark.parametrize("K,V,cu", [(128, 128, None), (64, 128, None), (128, 64, [0, 100, 700, 1500, 2100])])
def test_segment_scan_slow_gates(L, K, V, cu, monkeypatch):
    B, T, H = 1, 2100, 2
    note(f"segment scan L={L} K={K} V={V} cu={cu}")
    monkeypatch.setenv("KAIROS_GDN_SEG_CHUNKS", L)
    n = len(cu) - 1 if cu else None
    x = slow_gate_inputs(B, T, H, K, V, seed=7 + K + V, n_states=n)
    o, ht = run_gpu(x, "bf16", cu=cu)
    check_against_oracle(x, "bf16", o, ht, cu=cu)


def test_fp32_against_recurrence():
    """fp32 compute (the stage kernels) against the fp64 token recurrence with slow gates."""
    B, T, H, K, V = 2, 700, 2, 64, 64
    note("fp32 stage path vs fp64 token recurrence")
    x = make_inputs(B, T, H, K, V, seed=3, dtype="fp32", h0_scale=0.5)
    x["g"] = (x["g"] * 0.004).astype(np.float32)
    o, ht = run_gpu(x, "fp32")
    on, hn = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"])
    eo, eh = rel(host(o), on), rel(host(ht), hn)
    note(f"    rel-L2 o={eo:.2e} ht={eh:.2e}")
    assert eo < 1e-4 and eh < 1e-4


# ---------------------------------------------------------------------------
# config 4: streaming frame-by-frame rollout with fp8 q/k
# ---------------------------------------------------------------------------
@pytest.mark.skipif(not hasattr(torch, "float8_e4m3fn"), reason="torch without float8_e4m3fn")
def test_fp8_decode_every_code():
    """Every finite e4m3 code through the fused path: with g = 0, beta = 0, h0 = I and scale = 1 the
    output is q itself, o[t][d] = q[t][d], so o (bf16, exact for e4m3 values) must equal the decoded
    codes bit for bit (oracle fp8_e4m3_decode).  NaN codes (0x7f, 0xff) are replaced by 0: one NaN
    would reach every column through the 0 * NaN products of q h."""
    note("fp8 e4m3: every code decoded exactly")
    codes = np.arange(256, dtype=np.uint8).reshape(1, 2, 1, 128)
    codes[(codes & 0x7f) == 0x7f] = 0
    B, T, H, K, V = 1, 2, 1, 128, 128
    q8 = torch.from_numpy(codes).to("cuda").view(torch.float8_e4m3fn)
    k8 = torch.zeros(B, T, H, K, dtype=torch.uint8, device="cuda").view(torch.float8_e4m3fn)
    v = torch.randn(B, T, H, V, device="cuda").to(torch.bfloat16)
    g = torch.zeros(B, T, H, device="cuda")
    beta = torch.zeros(B, T, H, device="cuda", dtype=torch.bfloat16)
    h0 = torch.eye(K, device="cuda").reshape(1, 1, K, V)
    one = torch.ones(H, device="cuda")
    o, _ = kairos_gdn.chunk_gated_delta_rule(q8, k8, v, g, beta, scale=1.0, initial_state=h0,
                                             output_final_state=True, q_scale=one, k_scale=one)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(o).reshape(2, 128), O.fp8_e4m3_decode(codes).reshape(2, 128))


@pytest.mark.skipif(not hasattr(torch, "float8_e4m3fn"), reason="torch without float8_e4m3fn")
def test_fp8_qk_model_head_dims():
    """fp8 q/k at dk=256, dv=512 (the fused recurrence + output of the stage path), varlen."""
    B, T, H, K, V = 1, 300, 2, 256, 512
    cu = [0, 130, 300]
    note(f"fp8 q/k B={B} T={T} H={H} K={K} V={V} cu={cu}")
    x = make_inputs(B, T, H, K, V, seed=31, dtype="bf16", n_states=2)
    qc, qs = quantize_fp8(x["q"])
    kc, ks = quantize_fp8(x["k"])
    d = to_dev(x, "bf16")
    q8 = torch.from_numpy(qc).to("cuda").view(torch.float8_e4m3fn)
    k8 = torch.from_numpy(kc).to("cuda").view(torch.float8_e4m3fn)
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda")
    o, ht = kairos_gdn.chunk_gated_delta_rule(q8, k8, d["v"], d["g"], d["beta"], initial_state=d["h0"],
                                              output_final_state=True, cu_seqlens=cu_t, q_scale=dev(qs),
                                              k_scale=dev(ks))
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16
    xd = dict(x, q=dequant_bf16(qc, qs), k=dequant_bf16(kc, ks))
    check_against_oracle(xd, "bf16", o, ht, cu=cu)


@pytest.mark.skipif(not hasattr(torch, "float8_e4m3fn"), reason="torch without float8_e4m3fn")
def test_streaming_fp8_rollout():
    """Config 4: 21 calls of T = 1560 with the fp32 state carried, fp8 q/k.  Every frame's o and state on
    every head against the oracle run from the same input state (child processes over frames and head
    groups, tests/oracle_pool.py), and the end state's drift against one unquantised fp32 call."""
    import oracle_pool
    B, H, K, V, Tf, frames = 8, 20, 128, 128, 1560, 21
    seed = 20264
    note(f"config 4: B={B} H={H} {frames} calls of T={Tf}, fp8 q/k")
    dheads = [0, 7, 13, 19]                   # end-state drift (the fp32 single call over all frames)
    h0 = (0.02 * np.random.default_rng(seed).standard_normal((B, H, K, V))).astype(np.float32)
    state = dev(h0)
    S_in = h0[:, dheads]
    parts = []
    with oracle_pool.Scratch() as sc:
        for f in range(frames):
            x = make_inputs(B, Tf, H, K, V, seed=(seed, f), dtype="bf16", h0_scale=0.0)
            qc, qs = quantize_fp8(x["q"])
            kc, ks = quantize_fp8(x["k"])
            q8 = torch.from_numpy(qc).to("cuda").view(torch.float8_e4m3fn)
            k8 = torch.from_numpy(kc).to("cuda").view(torch.float8_e4m3fn)
            d = to_dev(x, "bf16")
            o, new_state = kairos_gdn.chunk_gated_delta_rule(q8, k8, d["v"], d["g"], d["beta"], initial_state=state,
                                                             output_final_state=True, q_scale=dev(qs),
                                                             k_scale=dev(ks))
            torch.cuda.synchronize()
            assert o.dtype == torch.bfloat16
            sc.put(f"o{f}", host(o), bf16=True)
            sc.put(f"si{f}", host(state))
            sc.put(f"so{f}", host(new_state))
            parts.append({k_: x[k_][:, :, dheads] for k_ in ("q", "k", "v", "g", "beta")})
            state = new_state
        note("    GPU rollout done; oracle per frame on every head")
        e = oracle_pool.run_heads(oracle_pool.fp8_frame_job, sc, H, group=10, workers=8, log=lambda m: None,
                                  kw=dict(shape=(B, Tf, H, K, V), seed=seed, frames=frames), frames=frames)
    for f in range(frames):
        note(f"    frame {f}: rel-L2 o={e[f'o{f}']:.3e} state={e[f'h{f}']:.3e}")
    assert all(e[f"o{f}"] < 1e-2 and e[f"h{f}"] < 5e-3 for f in range(frames))
    torch.cuda.synchronize()
    # drift of the streamed end state against one fp32 call over all 21 frames (unquantised q/k): the
    # e4m3 rounding of q and k (3 mantissa bits) bounds it; measured 2.7e-2
    cat = {k_: np.concatenate([p_[k_] for p_ in parts], axis=1) for k_ in parts[0]}
    _, h_single = O.chunk_gated_delta_rule(cat["q"], cat["k"], cat["v"], cat["g"], cat["beta"],
                                           initial_state=S_in, output_final_state=True, dtype="fp32")
    drift = rel(host(state)[:, dheads], h_single)
    note(f"    end-state drift vs single-call fp32 (unquantised q/k): {drift:.3e}")
    assert math.isfinite(drift) and drift < 0.05
