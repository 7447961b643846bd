"""Layer prologue: short causal convolution (ShortConvolution / causal_conv1d) and gates.

CPU: pins the oracle's ``causal_conv1d`` against torch.nn.functional.conv1d
(fp64) and its cache semantics, and ``gdn_gates`` against torch's softplus /
sigmoid.  GPU (``-m gpu``): the HIP kernels against the oracle through the C
ABI.  Tolerances (relative L2): y bf16 1e-2 (fp32 accumulation, one bf16
rounding; in practice ~1e-3), fp32 1e-5; final cache bit-exact (a copy of
inputs); gates: g 1e-5, beta bf16 1e-2 / fp32 1e-6.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O

rel = O.rel_l2


def conv_case(B, T, D, W, seed, N=None, cache=True, dtype="bf16"):
    rng = np.random.default_rng(seed)
    x = O.cast(rng.standard_normal((B, T, D)).astype(np.float32), dtype)
    w = O.cast((rng.standard_normal((D, W)) * 0.5).astype(np.float32), dtype)
    b = O.cast((rng.standard_normal(D) * 0.1).astype(np.float32), dtype)
    h0 = O.cast(rng.standard_normal((N or B, D, W)).astype(np.float32), dtype) if cache else None
    return x, w, b, h0


def torch_conv(x, w, b):
    """Causal depthwise conv by the library routine (fp64), no cache."""
    B, T, D = x.shape
    W = w.shape[1]
    xt = torch.from_numpy(np.asarray(x, np.float64)).transpose(1, 2)
    y = torch.nn.functional.conv1d(xt, torch.from_numpy(np.asarray(w, np.float64))[:, None, :],
                                   torch.from_numpy(np.asarray(b, np.float64)), padding=W - 1, groups=D)
    return y[..., :T].transpose(1, 2).numpy()


# ---------------------------------------------------------------------------
# oracle pinning (CPU)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("W", [2, 3, 4])
def test_conv_equals_torch_conv1d(W):
    x, w, b, _ = conv_case(2, 40, 24, W, seed=W, cache=False, dtype="fp32")
    y, _ = O.causal_conv1d(x, w, b, dtype="fp32")
    np.testing.assert_allclose(y, torch_conv(x, w, b), rtol=1e-5, atol=1e-6)
    ys, _ = O.causal_conv1d(x, w, b, activation="silu", dtype="fp32")
    z = torch.from_numpy(torch_conv(x, w, b))
    np.testing.assert_allclose(ys, torch.nn.functional.silu(z).numpy(), rtol=1e-5, atol=1e-6)


def test_conv_cache_split_calls_and_final_state():
    x, w, b, h0 = conv_case(1, 50, 16, 4, seed=5, dtype="fp32")
    y, hf = O.causal_conv1d(x, w, b, initial_state=h0, activation="silu", dtype="fp32")
    for cut in (1, 2, 3, 17):                                 # shorter and longer than W
        y1, h1 = O.causal_conv1d(x[:, :cut], w, b, initial_state=h0, activation="silu", dtype="fp32")
        y2, h2 = O.causal_conv1d(x[:, cut:], w, b, initial_state=h1, activation="silu", dtype="fp32")
        np.testing.assert_array_equal(np.concatenate([y1, y2], 1), y)
        np.testing.assert_array_equal(h2, hf)
    np.testing.assert_array_equal(hf[0], x[0, -4:].T)                         # T >= W: the last W inputs
    _, hs = O.causal_conv1d(x[:, :2], w, b, initial_state=h0, dtype="fp32")  # T < W: shifted cache + x
    np.testing.assert_array_equal(hs[0], np.concatenate([h0[0][:, 2:], x[0, :2].T], axis=1))
    # no cache: zeros before the first token
    _, hz = O.causal_conv1d(x[:, :1], w, b, dtype="fp32")
    np.testing.assert_array_equal(hz[0], np.concatenate([np.zeros((16, 3)), x[0, :1].T], axis=1))


def test_conv_varlen_equals_separate_calls():
    cu = np.array([0, 3, 3, 40, 64])
    x, w, b, h0 = conv_case(1, 64, 16, 4, seed=6, N=4, dtype="fp32")
    y, hf = O.causal_conv1d(x, w, b, initial_state=h0, cu_seqlens=cu, activation="silu", dtype="fp32")
    for n in range(4):
        yn, hn = O.causal_conv1d(x[:, cu[n]:cu[n + 1]], w, b, initial_state=h0[n:n + 1], activation="silu",
                                 dtype="fp32")
        np.testing.assert_array_equal(y[:, cu[n]:cu[n + 1]], yn)
        np.testing.assert_array_equal(hf[n:n + 1], hn)


def test_conv_planted_reversed_taps_fail():
    x, w, b, _ = conv_case(1, 30, 8, 4, seed=7, cache=False, dtype="fp32")
    y, _ = O.causal_conv1d(x, w[:, ::-1], b, dtype="fp32")
    assert rel(y, torch_conv(x, w, b)) > 1e-2


def test_conv_l2norm_fusion_equals_separate_norm():
    x, w, b, h0 = conv_case(1, 20, 256, 4, seed=8)
    y, _ = O.causal_conv1d(x, w, b, initial_state=h0, activation="silu", dtype="bf16")
    yl, _ = O.causal_conv1d(x, w, b, initial_state=h0, activation="silu", l2norm_head_dim=128, dtype="bf16")
    ref = O.l2norm(y.reshape(1, 20, 2, 128), dtype="bf16").reshape(1, 20, 256)
    np.testing.assert_array_equal(yl, ref)


def test_gates_against_torch():
    rng = np.random.default_rng(9)
    a = (rng.standard_normal((7, 5)) * 8).astype(np.float32)
    a[0, 0] = 25.0                                            # above the softplus threshold
    b = rng.standard_normal((7, 5)).astype(np.float32)
    A_log = np.log(rng.uniform(0, 16, 5)).astype(np.float32)
    dt = rng.standard_normal(5).astype(np.float32)
    g, beta = O.gdn_gates(a, b, A_log, dt)
    tg = -torch.from_numpy(A_log).double().exp() * torch.nn.functional.softplus(torch.from_numpy(a + dt).double())
    np.testing.assert_allclose(g, tg.numpy(), rtol=1e-6)
    np.testing.assert_allclose(beta, torch.sigmoid(torch.from_numpy(b).double()).numpy(), rtol=1e-6)
    g0, _ = O.gdn_gates(-dt[None], b[:1], A_log, dt)         # a + dt_bias = 0: softplus = log 2
    np.testing.assert_allclose(g0[0], -np.exp(A_log) * np.log(2.0), rtol=1e-6)
    _, b2 = O.gdn_gates(a, b, A_log, dt, allow_neg_eigval=True)
    np.testing.assert_array_equal(b2, 2 * beta)


# ---------------------------------------------------------------------------
# GPU parity through the C ABI
# ---------------------------------------------------------------------------
def _dev(a, dt=torch.float32):
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)


CONV_CASES = [
    # id, B, T, D, W, cu, cache, dtype, l2 head dim
    ("q_model_l2", 1, 300, 5120, 4, None, True, "bf16", 256),
    ("v_model", 1, 130, 10240, 4, None, False, "bf16", 0),
    ("varlen_empty", 1, 100, 640, 4, [0, 2, 2, 37, 100], True, "bf16", 128),
    ("batch_fp32_w3", 3, 45, 72, 3, None, True, "fp32", 0),
    ("w2_ragged_d", 2, 33, 520, 2, None, True, "bf16", 0),
    ("decode", 8, 1, 1024, 4, None, True, "bf16", 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("cid,B,T,D,W,cu,cache,dt,l2", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_gpu_causal_conv1d(cid, B, T, D, W, cu, cache, dt, l2):
    import kairos_gdn
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print(f"causal_conv1d {cid}: B={B} T={T} D={D} W={W} cu={cu} cache={cache} {dt} l2={l2}", flush=True)
    sys.stdout.flush()
    N = len(cu) - 1 if cu else B
    x, w, b, h0 = conv_case(B, T, D, W, seed=D + T, N=N, cache=cache, dtype=dt)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    y, hf = kairos_gdn.causal_conv1d(_dev(x, tdt), _dev(w, tdt), _dev(b, tdt), initial_state=_dev(h0, tdt),
                                     output_final_state=True, activation="silu", cu_seqlens=cu_t,
                                     l2norm_head_dim=l2)
    torch.cuda.synchronize()
    y_r, h_r = O.causal_conv1d(x, w, b, initial_state=h0, cu_seqlens=np.array(cu) if cu else None,
                               activation="silu", l2norm_head_dim=l2, dtype=dt)
    e = rel(y.float().cpu().numpy(), y_r)
    print(f"    rel-L2 y={e:.3e}", flush=True)
    assert y.dtype == tdt and e < (1e-2 if dt == "bf16" else 1e-5)
    np.testing.assert_array_equal(hf.float().cpu().numpy(), h_r)


@pytest.mark.gpu
def test_gpu_short_convolution_module_prefill_then_decode():
    import kairos_gdn
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("ShortConvolution prefill + 3 decode steps", flush=True)
    torch.manual_seed(0)
    D, W, B = 256, 4, 2
    conv = kairos_gdn.ShortConvolution(D, W, bias=False, activation="silu").to("cuda", torch.bfloat16)
    x = torch.randn(B, 40, D).to("cuda", torch.bfloat16)
    y_all, _ = conv(x)
    y, cache = conv(x[:, :37], output_final_state=True)
    outs = [y]
    for t in range(37, 40):                                   # one token per sequence: cache updated in place
        c0 = cache.data_ptr()
        yt, cache = conv(x[:, t:t + 1], cache=cache, output_final_state=True)
        assert cache.data_ptr() == c0
        outs.append(yt)
    torch.cuda.synchronize()
    torch.testing.assert_close(torch.cat(outs, 1), y_all, rtol=0, atol=0)


@pytest.mark.gpu
def test_gpu_inference_mode_cu_seqlens():
    """cu_seqlens made under torch.inference_mode() (no version counter), as a serving loop builds it:
    the chunked forward and ShortConvolution both run and match the same calls with an ordinary tensor."""
    import kairos_gdn
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("inference-mode cu_seqlens: chunk forward + ShortConvolution", flush=True)
    torch.manual_seed(1)
    T, H, K, D = 200, 2, 64, 128
    cu_list = [0, 70, 71, 200]
    q = torch.nn.functional.normalize(torch.randn(1, T, H, K), dim=-1).to("cuda", torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn(1, T, H, K), dim=-1).to("cuda", torch.bfloat16)
    v = torch.randn(1, T, H, K).to("cuda", torch.bfloat16)
    g = -torch.nn.functional.softplus(torch.randn(1, T, H)).to("cuda")
    beta = torch.sigmoid(torch.randn(1, T, H)).to("cuda", torch.bfloat16)
    x = torch.randn(1, T, D).to("cuda", torch.bfloat16)
    conv = kairos_gdn.ShortConvolution(D, 4, bias=False, activation="silu").to("cuda", torch.bfloat16)
    cu_plain = torch.tensor(cu_list, dtype=torch.int64, device="cuda")
    with torch.no_grad():
        o_ref, _ = kairos_gdn.chunk_gated_delta_rule(q, k, v, g, beta, cu_seqlens=cu_plain)
        y_ref, _ = conv(x, cu_seqlens=cu_plain)
    with torch.inference_mode():
        cu_inf = torch.tensor(cu_list, dtype=torch.int64, device="cuda")
        assert cu_inf.is_inference()
        for _ in range(2):                                    # the second call finds nothing cached
            o, _ = kairos_gdn.chunk_gated_delta_rule(q, k, v, g, beta, cu_seqlens=cu_inf)
            y, _ = conv(x, cu_seqlens=cu_inf)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)
    assert torch.equal(y, y_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("bdt", ["bf16", "fp32"])
def test_gpu_gates(bdt):
    import kairos_gdn
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print(f"gates b={bdt}", flush=True)
    rng = np.random.default_rng(10)
    rows, HV = 3000, 20
    a = O.cast((rng.standard_normal((rows, HV)) * 4).astype(np.float32), bdt)
    b = O.cast(rng.standard_normal((rows, HV)).astype(np.float32), bdt)
    a[0, 0] = 30.0
    A_log = np.log(rng.uniform(0, 16, HV)).astype(np.float32)
    dt = rng.standard_normal(HV).astype(np.float32)
    tdt = torch.bfloat16 if bdt == "bf16" else torch.float32
    for neg in (False, True):
        g, beta = kairos_gdn.gdn_gates(_dev(a, tdt), _dev(b, tdt), _dev(A_log), _dev(dt), allow_neg_eigval=neg)
        torch.cuda.synchronize()
        g_r, b_r = O.gdn_gates(a, b, A_log, dt, allow_neg_eigval=neg, b_dtype=bdt)
        assert g.dtype == torch.float32 and beta.dtype == tdt
        assert rel(g.cpu().numpy(), g_r) < 1e-5
        got = beta.float().cpu().numpy()
        if bdt == "bf16":
            # beta = sigmoid(b) rounded once to bf16: at most one bf16 ulp of the oracle's rounding, and
            # bitwise equal but for the rare values whose fp32 sigmoid sits at a rounding boundary
            ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(b_r), 1e-30))) - 7)
            assert (np.abs(got - b_r) <= ulp).all()
            assert (got == b_r).mean() > 0.99
        else:
            assert rel(got, b_r) < 1e-6
