"""Pins the backward oracle (oracle/gdn_oracle_bwd.py) before it is trusted as the parity checker.

The reference ships no gradient fixtures, so the chunked backward restatement
is pinned by what the mathematics fixes: in fp64 it must equal torch autograd
through the fp64 token recurrence (a formulation with no chunks, no WY
representation and no hand-written derivative); that autograd is checked by
central finite differences of gdn_oracle.naive_recurrent; and planted
mistakes in the restatement must fail the check.  CPU only.
"""
import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
from oracle import gdn_oracle_bwd as OB
from gdn_inputs import make_inputs


def rec_torch(q, k, v, g, beta, scale, h0, spans, l2=False):
    """fp64 token recurrence in torch (gated_delta_product/naive.py:23-35), differentiable.
    spans: (batch_row, bos, eos) per sequence.  Returns (o [B,T,H,V], ht [N,H,K,V])."""
    if l2:
        q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    B, T, H, K = q.shape
    V = v.shape[-1]
    o_rows = [[None] * T for _ in range(B)]
    hts = []
    for n, (b, bos, eos) in enumerate(spans):
        S = h0[n] if h0 is not None else torch.zeros(H, K, V, dtype=q.dtype)
        for t in range(bos, eos):
            S = S * torch.exp(g[b, t])[:, None, None]
            kt = k[b, t]
            vp = beta[b, t][:, None] * (v[b, t] - torch.einsum("hkv,hk->hv", S, kt))
            S = S + kt[:, :, None] * vp[:, None, :]
            o_rows[b][t] = scale * torch.einsum("hkv,hk->hv", S, q[b, t])
        hts.append(S)
    zero = torch.zeros(H, V, dtype=q.dtype)
    o = torch.stack([torch.stack([r if r is not None else zero for r in row]) for row in o_rows])
    return o, torch.stack(hts)


def case(B, T, H, K, V, seed, cu=None, h0=True, dht=True, l2=False):
    x = make_inputs(B, T, H, K, V, seed, dtype="fp64", n_states=(len(cu) - 1 if cu else None),
                    h0_scale=0.5 if h0 else 0.0)
    x = {k_: (np.asarray(v_, np.float64) if v_ is not None else None) for k_, v_ in x.items()}
    rng = np.random.default_rng(seed + 1000)
    if l2:              # unnormalised q, k: the op normalises them
        x["q"] = x["q"] * rng.uniform(0.5, 3.0, x["q"].shape[:-1] + (1,))
        x["k"] = x["k"] * rng.uniform(0.5, 3.0, x["k"].shape[:-1] + (1,))
    else:
        for n in ("q", "k"):
            x[n] = x[n] / np.linalg.norm(x[n], axis=-1, keepdims=True)
    N = len(cu) - 1 if cu else B
    x["do"] = rng.standard_normal((B, T, H, V))
    x["dht"] = rng.standard_normal((N, H, K, V)) if dht else None
    x["cu"] = cu
    x["l2"] = l2
    return x


def autograd_grads(x):
    B, T, H, K = x["q"].shape
    spans = O.seq_spans(B, T, x["cu"])
    ts = {n: torch.tensor(x[n], dtype=torch.float64, requires_grad=True) for n in ("q", "k", "v", "g", "beta")}
    h0 = torch.tensor(x["h0"], dtype=torch.float64, requires_grad=True) if x["h0"] is not None else None
    o, ht = rec_torch(ts["q"], ts["k"], ts["v"], ts["g"], ts["beta"], K ** -0.5, h0, spans, l2=x["l2"])
    loss = (o * torch.tensor(x["do"])).sum()
    if x["dht"] is not None:
        loss = loss + (ht * torch.tensor(x["dht"])).sum()
    loss.backward()
    out = [ts[n].grad.numpy() for n in ("q", "k", "v", "g", "beta")]
    out.append(h0.grad.numpy() if h0 is not None else None)
    return out


def oracle_grads(x, dtype="fp64"):
    return OB.chunk_gated_delta_rule_bwd(x["q"], x["k"], x["v"], x["g"], x["beta"], x["do"], dht=x["dht"],
                                         initial_state=x["h0"], use_qk_l2norm_in_kernel=x["l2"],
                                         cu_seqlens=x["cu"], dtype=dtype)


NAMES = ("dq", "dk", "dv", "dg", "dbeta", "dh0")


def max_err(got, ref):
    errs = {}
    for n, a, b in zip(NAMES, got, ref):
        if b is None:
            assert a is None, n
            continue
        errs[n] = O.rel_l2(a, b)
    return errs


CASES = [
    dict(B=1, T=64, H=1, K=16, V=16),                                  # one full chunk
    dict(B=2, T=130, H=2, K=32, V=48),                                 # ragged tail, batch 2
    dict(B=1, T=150, H=2, K=16, V=32, cu=[0, 70, 71, 71, 150]),        # varlen: 1-token and empty sequences
    dict(B=1, T=100, H=2, K=16, V=16, h0=False, dht=False),            # no states
    dict(B=1, T=140, H=2, K=16, V=16, l2=True),                        # in-kernel L2 norm
]


@pytest.mark.parametrize("c", CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_fp64_backward_equals_autograd_of_recurrence(c):
    x = case(seed=5, **c)
    errs = max_err(oracle_grads(x), autograd_grads(x))
    assert all(e < 1e-9 for e in errs.values()), errs


def test_autograd_recurrence_matches_finite_differences():
    """The differentiable torch recurrence above is the numpy recurrence the forward oracle is pinned by:
    central differences of O.naive_recurrent's loss agree with its autograd on sampled coordinates."""
    x = case(1, 70, 2, 8, 8, seed=9)
    grads = autograd_grads(x)
    rng = np.random.default_rng(3)

    def loss(xx):
        o, ht = O.naive_recurrent(xx["q"], xx["k"], xx["v"], xx["g"], xx["beta"], initial_state=xx["h0"])
        return float((o * xx["do"]).sum() + (ht * xx["dht"]).sum())

    for gi, n in enumerate(("q", "k", "v", "g", "beta", "h0")):
        for _ in range(3):
            idx = tuple(rng.integers(0, s) for s in x[n].shape)
            eps = 1e-6
            xp = dict(x, **{n: x[n].copy()})
            xm = dict(x, **{n: x[n].copy()})
            xp[n][idx] += eps
            xm[n][idx] -= eps
            fd = (loss(xp) - loss(xm)) / (2 * eps)
            assert abs(fd - grads[gi][idx]) < 1e-6 * max(1.0, abs(fd)), (n, idx, fd, grads[gi][idx])


def _no_reverse_cumsum(dgc, cm):
    return np.where(cm.valid[:, None, :], dgc, 0.0)


def _dropped_kkt_term(cm, kc, vc, bc, Aic, gcc, dwc, duc, f, dtype):
    dk, dv, db, dg = ORIG_WY(cm, kc, vc, bc, Aic, gcc, dwc, duc, f, dtype)
    return dk, dv, db, np.zeros_like(dg)


def _undecayed_dh(cm, qc, kc, wc, doc, dvc, gcc, scale, h0, dht, f, dtype):
    return ORIG_DHU(cm, qc, kc, wc, doc, dvc, np.zeros_like(gcc), scale, h0, dht, f, dtype)


def _strict_dv_local(cm, qc, kc, doc, gcc, scale, f, dtype):
    m = np.swapaxes(O._pair_mask(cm, True), -1, -2)
    At = (kc @ np.swapaxes(qc, -1, -2)) * scale * np.exp(np.where(m, gcc[..., None, :] - gcc[..., :, None], 0.0))
    return np.where(m, At, 0.0) @ doc


ORIG_WY = OB._wy_bwd_c
ORIG_DHU = OB._dhu_c


@pytest.mark.parametrize("target,replacement", [
    ("reverse_chunk_cumsum", _no_reverse_cumsum),
    ("_wy_bwd_c", _dropped_kkt_term),
    ("_dhu_c", _undecayed_dh),
    ("_dv_local_c", _strict_dv_local),
])
def test_planted_mistake_is_caught(monkeypatch, target, replacement):
    x = case(1, 130, 2, 16, 16, seed=13)
    ref = autograd_grads(x)
    monkeypatch.setattr(OB, target, replacement)
    errs = max_err(oracle_grads(x), ref)
    assert max(errs.values()) > 1e-3, (target, errs)


def test_bf16_cast_points_stay_near_fp64():
    """The bf16 restatement (the GPU parity target) stays close to the exact gradients."""
    x = case(1, 200, 2, 64, 64, seed=17)
    xb = dict(x)
    for n in ("q", "k", "v", "beta", "do"):
        xb[n] = O.to_bf16(x[n])
    xb["g"] = x["g"].astype(np.float32)
    ref = oracle_grads(xb, dtype="fp64")
    got = oracle_grads(xb, dtype="bf16")
    errs = max_err(got, ref)
    assert all(e < 2e-2 for e in errs.values()), errs
