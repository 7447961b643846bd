"""Pins the CPU oracle (oracle/gdn_oracle.py) before it is trusted as the parity checker.

The reference ships no golden vectors for this op, so each oracle function is
pinned by what the mathematics fixes: closed forms, brute force on tiny
inputs, the fp64 token recurrence, invariants, and planted mistakes that must
fail those checks.  All CPU; no GPU, no reference code is run.
"""
import numpy as np
import pytest

from oracle import gdn_oracle as O
from gdn_inputs import make_inputs


def rand_case(B, T, H, K, V, seed, cu=None, h0=True):
    x = make_inputs(B, T, H, K, V, seed, dtype="fp64", n_states=(len(cu) - 1 if cu is not None else None),
                    h0_scale=0.5 if h0 else 0.0)
    x = {k_: (v_.astype(np.float64) if v_ is not None else None) for k_, v_ in x.items()}
    for name in ("q", "k"):                              # unit norm in fp64
        x[name] = x[name] / np.linalg.norm(x[name], axis=-1, keepdims=True)
    return x


def run_both(x, cu=None, chunk=64, scale=None):
    o, ht = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], scale=scale, initial_state=x["h0"],
                                     output_final_state=True, cu_seqlens=cu, chunk=chunk, dtype="fp64")
    on, hn = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], scale=scale, initial_state=x["h0"],
                               cu_seqlens=cu)
    return o, ht, on, hn


# ---------------------------------------------------------------------------
# cumsum
# ---------------------------------------------------------------------------
def test_cumsum_closed_form_varlen():
    rng = np.random.default_rng(1)
    cu = [0, 5, 5, 70, 200, 201]
    g = rng.standard_normal((1, 201, 3)).astype(np.float32)
    gc = O.chunk_local_cumsum(g, cu_seqlens=np.array(cu))
    exp = np.zeros_like(g)
    for s in range(len(cu) - 1):
        for t in range(cu[s], cu[s + 1]):
            start = cu[s] + ((t - cu[s]) // 64) * 64
            exp[0, t] = g[0, start:t + 1].sum(axis=0)
    np.testing.assert_allclose(gc, exp, rtol=1e-5, atol=1e-5)


def test_cumsum_fixed_batch_restarts():
    g = np.ones((2, 130, 1), np.float32)
    gc = O.chunk_local_cumsum(g)
    expect = np.concatenate([np.arange(1, 65), np.arange(1, 65), np.arange(1, 3)]).astype(np.float32)
    np.testing.assert_array_equal(gc[0, :, 0], expect)
    np.testing.assert_array_equal(gc[1, :, 0], expect)


# ---------------------------------------------------------------------------
# K.K^T and the triangular solve
# ---------------------------------------------------------------------------
def test_kkt_bruteforce():
    x = rand_case(1, 90, 2, 8, 8, seed=2)
    gc = O.chunk_local_cumsum(x["g"], dtype="fp64")
    A = O.chunk_scaled_dot_kkt(x["k"], gc, x["beta"], dtype="fp64")
    exp = np.zeros_like(A)
    for h in range(2):
        for t in range(90):
            c0 = (t // 64) * 64
            for j in range(c0, t):
                exp[0, t, h, j - c0] = x["beta"][0, t, h] * np.exp(gc[0, t, h] - gc[0, j, h]) * \
                    np.dot(x["k"][0, t, h], x["k"][0, j, h])
    np.testing.assert_allclose(A, exp, rtol=1e-12, atol=1e-14)


def test_solve_tril_is_inverse():
    rng = np.random.default_rng(3)
    T, H = 150, 2
    A = np.zeros((1, T, H, 64))
    for t in range(T):
        c0 = (t // 64) * 64
        A[0, t, :, :t - c0] = 0.3 * rng.standard_normal((H, t - c0))
    Ai = O.solve_tril(A, dtype="fp64")
    for c0 in range(0, T, 64):
        n = min(64, T - c0)
        for h in range(H):
            L = A[0, c0:c0 + n, h, :n]
            X = Ai[0, c0:c0 + n, h, :n]
            np.testing.assert_allclose(X, np.linalg.inv(np.eye(n) + L), rtol=1e-9, atol=1e-9)
            np.testing.assert_allclose((np.eye(n) + L) @ X, np.eye(n), atol=1e-9)


def test_w_u_definition():
    x = rand_case(1, 70, 2, 8, 6, seed=4)
    gc = O.chunk_local_cumsum(x["g"], dtype="fp64")
    A = O.chunk_scaled_dot_kkt(x["k"], gc, x["beta"], dtype="fp64")
    Ai = O.solve_tril(A, dtype="fp64")
    w, u = O.recompute_w_u(x["k"], x["v"], x["beta"], Ai, gc, dtype="fp64")
    for c0 in (0, 64):
        n = min(64, 70 - c0)
        for h in range(2):
            X = Ai[0, c0:c0 + n, h, :n]
            b = x["beta"][0, c0:c0 + n, h][:, None]
            np.testing.assert_allclose(u[0, c0:c0 + n, h], X @ (x["v"][0, c0:c0 + n, h] * b), rtol=1e-12, atol=1e-12)
            e = np.exp(gc[0, c0:c0 + n, h])[:, None]
            np.testing.assert_allclose(w[0, c0:c0 + n, h], X @ (x["k"][0, c0:c0 + n, h] * b * e), rtol=1e-12,
                                       atol=1e-12)


# ---------------------------------------------------------------------------
# the token recurrence itself (closed forms)
# ---------------------------------------------------------------------------
def test_naive_beta_zero_is_pure_decay():
    x = rand_case(1, 20, 2, 4, 3, seed=5)
    x["beta"] = np.zeros_like(x["beta"])
    o, ht = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], scale=0.7, initial_state=x["h0"])
    S = x["h0"][0].copy()
    for t in range(20):
        S = S * np.exp(x["g"][0, t])[:, None, None]
        np.testing.assert_allclose(o[0, t], 0.7 * np.einsum("hkv,hk->hv", S, x["q"][0, t]), rtol=1e-12)
    np.testing.assert_allclose(ht[0], S, rtol=1e-12)


def test_naive_exact_recall():
    # beta = 1, g = 0, unit k: after writing (k_t, v_t) the state recalls v_t exactly
    x = rand_case(1, 6, 1, 8, 5, seed=6)
    x["beta"] = np.ones_like(x["beta"])
    x["g"] = np.zeros_like(x["g"])
    for t in range(6):
        _, ht = O.naive_recurrent(x["q"][:, :t + 1], x["k"][:, :t + 1], x["v"][:, :t + 1], x["g"][:, :t + 1],
                                  x["beta"][:, :t + 1], initial_state=x["h0"])
        np.testing.assert_allclose(ht[0, 0].T @ x["k"][0, t, 0], x["v"][0, t, 0], rtol=1e-10, atol=1e-12)


def test_naive_two_token_scalar_by_hand():
    q = np.array([2.0, -1.0]).reshape(1, 2, 1, 1)
    k = np.array([1.0, 0.5]).reshape(1, 2, 1, 1)
    v = np.array([3.0, 4.0]).reshape(1, 2, 1, 1)
    g = np.log(np.array([0.5, 0.25])).reshape(1, 2, 1)
    beta = np.array([0.5, 1.0]).reshape(1, 2, 1)
    h0 = np.array([[[[2.0]]]])
    o, ht = O.naive_recurrent(q, k, v, g, beta, scale=1.0, initial_state=h0)
    # t0: S = 0.5*2 = 1; v' = 0.5*(3 - 1*1) = 1; S = 1 + 1*1 = 2; o = 2*2 = 4
    # t1: S = 0.25*2 = 0.5; v' = 1*(4 - 0.5*0.5) = 3.75; S = 0.5 + 0.5*3.75 = 2.375; o = -2.375
    np.testing.assert_allclose(o.ravel(), [4.0, -2.375])
    np.testing.assert_allclose(ht.ravel(), [2.375])


# ---------------------------------------------------------------------------
# chunked form == token recurrence (fp64), plus invariants
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,T,H,K,V,cu", [
    (1, 200, 2, 16, 24, None),
    (2, 64, 2, 8, 8, None),
    (2, 130, 3, 16, 16, None),
    (1, 1, 1, 8, 8, None),
    (1, 63, 2, 8, 16, None),
    (1, 300, 2, 16, 8, [0, 37, 37, 101, 229, 300]),
])
def test_chunked_equals_recurrence_fp64(B, T, H, K, V, cu):
    x = rand_case(B, T, H, K, V, seed=T + K, cu=cu)
    o, ht, on, hn = run_both(x, cu=np.array(cu) if cu else None)
    assert O.rel_l2(o, on) < 1e-10
    assert O.rel_l2(ht, hn) < 1e-10


def test_chunk_size_independence():
    x = rand_case(1, 150, 2, 16, 16, seed=7)
    outs = [O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                     output_final_state=True, chunk=c, dtype="fp64") for c in (16, 32, 64)]
    for o, ht in outs[1:]:
        assert O.rel_l2(o, outs[0][0]) < 1e-11 and O.rel_l2(ht, outs[0][1]) < 1e-11


def test_split_calls_with_state_carry():
    x = rand_case(1, 200, 2, 16, 8, seed=8)
    o, ht = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                     output_final_state=True, dtype="fp64")
    s = 77
    p1 = {k_: v_[:, :s] for k_, v_ in x.items() if k_ != "h0"}
    p2 = {k_: v_[:, s:] for k_, v_ in x.items() if k_ != "h0"}
    o1, h1 = O.chunk_gated_delta_rule(p1["q"], p1["k"], p1["v"], p1["g"], p1["beta"], initial_state=x["h0"],
                                      output_final_state=True, dtype="fp64")
    o2, h2 = O.chunk_gated_delta_rule(p2["q"], p2["k"], p2["v"], p2["g"], p2["beta"], initial_state=h1,
                                      output_final_state=True, dtype="fp64")
    assert O.rel_l2(np.concatenate([o1, o2], axis=1), o) < 1e-11
    assert O.rel_l2(h2, ht) < 1e-11


def test_varlen_equals_separate_calls():
    cu = [0, 40, 140, 141, 260]
    x = rand_case(1, 260, 2, 8, 8, seed=9, cu=cu)
    o, ht = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                     output_final_state=True, cu_seqlens=np.array(cu), dtype="fp64")
    for n in range(len(cu) - 1):
        sl = slice(cu[n], cu[n + 1])
        on, hn = O.chunk_gated_delta_rule(x["q"][:, sl], x["k"][:, sl], x["v"][:, sl], x["g"][:, sl],
                                          x["beta"][:, sl], initial_state=x["h0"][n:n + 1], output_final_state=True,
                                          dtype="fp64")
        np.testing.assert_allclose(o[:, sl], on, rtol=1e-11, atol=1e-13)
        np.testing.assert_allclose(ht[n:n + 1], hn, rtol=1e-11, atol=1e-13)


def test_linear_in_v_and_h0():
    x1 = rand_case(1, 100, 2, 8, 8, seed=10)
    x2 = rand_case(1, 100, 2, 8, 8, seed=11)
    common = dict(q=x1["q"], k=x1["k"], g=x1["g"], beta=x1["beta"])
    a, b = 0.7, -1.3
    f = lambda v, h0: O.chunk_gated_delta_rule(common["q"], common["k"], v, common["g"], common["beta"],  # noqa: E731
                                               initial_state=h0, output_final_state=True, dtype="fp64")
    o1, h1 = f(x1["v"], x1["h0"])
    o2, h2 = f(x2["v"], x2["h0"])
    o3, h3 = f(a * x1["v"] + b * x2["v"], a * x1["h0"] + b * x2["h0"])
    assert O.rel_l2(o3, a * o1 + b * o2) < 1e-11
    assert O.rel_l2(h3, a * h1 + b * h2) < 1e-11


def test_causality_of_ragged_tail():
    x = rand_case(1, 128, 2, 8, 8, seed=12)
    o_full, _ = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                         dtype="fp64")
    o_part, _ = O.chunk_gated_delta_rule(x["q"][:, :100], x["k"][:, :100], x["v"][:, :100], x["g"][:, :100],
                                         x["beta"][:, :100], initial_state=x["h0"], dtype="fp64")
    np.testing.assert_allclose(o_part, o_full[:, :100], rtol=1e-12, atol=1e-14)


def test_gate_reset():
    x = rand_case(1, 70, 1, 8, 4, seed=13)
    x["g"][0, -1] = -1e4                       # state forgotten right before the last write
    _, ht = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                     output_final_state=True, dtype="fp64")
    expect = x["beta"][0, -1, 0] * np.outer(x["k"][0, -1, 0], x["v"][0, -1, 0])
    np.testing.assert_allclose(ht[0, 0], expect, rtol=1e-10, atol=1e-12)


def test_bf16_cast_points_stay_within_tolerance():
    x = make_inputs(1, 300, 2, 64, 64, seed=14, dtype="bf16")
    o, ht = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                     output_final_state=True, dtype="bf16")
    on, hn = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"])
    assert O.rel_l2(o, on) < 1e-2
    assert O.rel_l2(ht, hn) < 5e-3


# ---------------------------------------------------------------------------
# planted mistakes: each must fail the recurrence check
# ---------------------------------------------------------------------------
def _wrong_solve(Ac, f):
    return _orig_solve(-np.asarray(Ac), f)                    # (I - A)^-1 instead of (I + A)^-1


def _strict_mask_fwd_o(cm, qc, kc, vnc, h, gcc, scale, f, dtype):
    o1 = (qc @ np.asarray(h, f)) * np.exp(gcc)[..., None]
    m = O._pair_mask(cm, True)
    diff = np.where(m, gcc[..., :, None] - gcc[..., None, :], 0.0)
    Aqk = np.where(m, (qc @ np.swapaxes(kc, 2, 3)) * np.exp(diff), 0.0)
    return o1 * scale + (Aqk @ vnc) * scale


def _decayed_vnew_fwd_h(cm, kc, wc, uc, gcc, initial_state, f, dtype):
    h, vnew, ht = _orig_fwd_h(cm, kc, wc, uc, gcc, initial_state, f, dtype)
    last = np.take_along_axis(gcc, (cm.nv - 1)[:, None, None].repeat(gcc.shape[1], 1), axis=2)
    return h, vnew * np.exp(last - gcc)[..., None], ht


def _no_beta_wu(kc, vc, bc, Aic, gcc, f, dtype):
    w, _ = _orig_wu(kc, vc, bc, Aic, gcc, f, dtype)
    return w, Aic @ vc


_orig_fwd_h = O._fwd_h_c
_orig_wu = O._wu_c
_orig_solve = O._solve_c


@pytest.mark.parametrize("target,replacement", [
    ("_solve_c", _wrong_solve),
    ("_fwd_o_c", _strict_mask_fwd_o),
    ("_fwd_h_c", _decayed_vnew_fwd_h),
    ("_wu_c", _no_beta_wu),
])
def test_planted_mistake_is_caught(monkeypatch, target, replacement):
    x = rand_case(1, 150, 2, 16, 16, seed=15)
    monkeypatch.setattr(O, target, replacement)
    o, ht, on, hn = run_both(x)
    assert O.rel_l2(o, on) > 1e-3


def test_planted_cumsum_without_sequence_restart_is_caught(monkeypatch):
    cu = np.array([0, 30, 150])
    x = rand_case(1, 150, 2, 8, 8, seed=16, cu=cu)

    orig_init = O.ChunkMap.__init__

    def bad_init(self, B, T, cu_seqlens=None, chunk=64):
        orig_init(self, B, T, cu_seqlens, chunk)
        if cu_seqlens is not None:                           # chunks aligned to 64 across the boundary
            idx = np.arange(0, -(-B * T // chunk) * chunk).reshape(-1, chunk)
            idx = np.where(idx < B * T, idx, B * T)
            self.idx, self.valid = idx, idx < B * T
            self.nv = self.valid.sum(axis=1)
            self.nc = idx.shape[0]
            self.chunk_offsets = [0] + [self.nc] * len(self.spans)
            self.spans = [(0, 0, B * T)] * len(self.spans)

    monkeypatch.setattr(O.ChunkMap, "__init__", bad_init)
    o, ht = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                     output_final_state=True, cu_seqlens=cu, dtype="fp64")
    monkeypatch.undo()
    on, hn = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"], cu_seqlens=cu)
    assert O.rel_l2(o, on) > 1e-3


# ---------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------
def test_l2norm_closed_form():
    x = np.array([[3.0, 4.0], [0.0, 0.0]], np.float32)
    y = O.l2norm(x)
    np.testing.assert_allclose(y[0], [0.6, 0.8], rtol=1e-6)
    np.testing.assert_array_equal(y[1], [0.0, 0.0])


def test_bf16_rounding_is_rtne():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 3.0e38], np.float32)
    out = O.to_bf16(vals)
    np.testing.assert_array_equal(out[:4], np.array([1.0, 1.0, 1.0 + 2 ** -6, -1.0], np.float32))
    assert np.isfinite(out[4])


def test_fp8_e4m3_codes():
    dec = O.fp8_e4m3_decode(np.array([0x38, 0x7E, 0x01, 0x08, 0xB8, 0x00], np.uint8))
    np.testing.assert_array_equal(dec, np.array([1.0, 448.0, 2.0 ** -9, 2.0 ** -6, -1.0, 0.0], np.float32))
    codes = np.arange(256, dtype=np.uint8)
    vals = O.fp8_e4m3_decode(codes)
    finite = np.isfinite(vals) & (codes != 0x80)
    np.testing.assert_array_equal(O.fp8_e4m3_quantize(vals[finite]), codes[finite])
    # ties go to the even code: halfway between 1.0 (0x38) and 1.125 (0x39)
    assert O.fp8_e4m3_quantize(np.array([1.0625]))[0] == 0x38


# ---------------------------------------------------------------------------
# the fp32 torch-CPU restatement timed as bench.py's CPU baseline
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,T,H,K,V,cu", [(2, 130, 3, 32, 48, None), (1, 150, 2, 64, 64, [0, 70, 71, 71, 150])])
def test_torch_cpu_restatement(B, T, H, K, V, cu):
    """oracle/gdn_torch_cpu.py: float64 == the fp64 token recurrence; float32 == the numpy fp32 oracle."""
    import torch
    from oracle import gdn_torch_cpu as TC
    x = rand_case(B, T, H, K, V, seed=41, cu=cu)
    t = lambda a, dt: torch.from_numpy(np.asarray(a)).to(dt)  # noqa: E731
    on, hn = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"], cu_seqlens=cu)
    args64 = [t(x[n], torch.float64) for n in ("q", "k", "v", "g", "beta")]
    o64, h64 = TC.chunk_gated_delta_rule(*args64, initial_state=t(x["h0"], torch.float64), cu_seqlens=cu)
    assert O.rel_l2(o64.numpy(), on) < 1e-10 and O.rel_l2(h64.numpy(), hn) < 1e-10
    args32 = [t(x[n], torch.float32) for n in ("q", "k", "v", "g", "beta")]
    o32, h32 = TC.chunk_gated_delta_rule(*args32, initial_state=t(x["h0"], torch.float32), cu_seqlens=cu)
    f32 = lambda a: np.asarray(a, np.float32)  # noqa: E731
    oo, ho = O.chunk_gated_delta_rule(*(f32(x[n]) for n in ("q", "k", "v", "g", "beta")),
                                      initial_state=f32(x["h0"]), output_final_state=True, cu_seqlens=cu, dtype="fp32")
    assert O.rel_l2(o32.numpy(), oo) < 1e-5 and O.rel_l2(h32.numpy(), ho) < 1e-5


def test_oracle_pool_combines_head_groups():
    """The child-process oracle used for full-size checks on every head (tests/oracle_pool.py) gives the
    single-process rel-L2: 0 for the oracle's own outputs, and the error of a planted change in one head."""
    import oracle_pool
    from gdn_inputs import make_inputs
    B, T, H, K, V = 1, 200, 5, 64, 64
    x = make_inputs(B, T, H, K, V, seed=5, dtype="bf16")
    o, ht = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                     output_final_state=True, dtype="bf16")
    e = oracle_pool.forward_all_heads(x, o, ht, "bf16", workers=2, group=2, log=lambda m: None)
    assert e["o"] == 0.0 and e["ht"] == 0.0
    o2 = o.copy()
    o2[:, :, 3] = O.to_bf16(o2[:, :, 3] * 1.5)                # a planted error in one head
    e2 = oracle_pool.forward_all_heads(x, o2, ht, "bf16", workers=2, group=2, log=lambda m: None)
    assert abs(e2["o"] - O.rel_l2(o2, o)) < 1e-6 and e2["o"] > 1e-2
