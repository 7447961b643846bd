"""CPU restatement of the chunked GatedDeltaNet BACKWARD -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module (the parity checker of the HIP backward
kernels); the product path never calls it.  It restates, stage by stage,
``chunk_gated_delta_rule_bwd`` of flash-linear-attention 0.4.0 as vendored in
``kairos/third_party/fla`` (paths below are relative to that tree), on the
chunked arrays and precision model of ``gdn_oracle``:

  stage                      reference
  -------------------------  ------------------------------------------------
  orchestration              ops/gated_delta_rule/chunk.py:70-146, backward :188-213
  recompute w, u, h, v_new   chunk.py:84-101 (wy_fast.py:55-81, chunk_delta_h.py:113-224)
  chunk_bwd_dv_local         ops/common/chunk_o.py:413-468, :585-628
  chunk_..._bwd_dhu          ops/common/chunk_delta_h.py:250-438, :504-556
  chunk_bwd_dqkwg            ops/common/chunk_o.py:147-326, :631-699
  prepare_wy_repr_bwd        ops/gated_delta_rule/wy_fast.py:98-210, :252-290
  reverse chunk cumsum       ops/utils/cumsum.py:58-63 (REVERSE)
  l2norm_bwd                 modules/l2norm.py:132-154, :203-240

Cast points ("bf16" mode), as the reference stores or converts: dv_local's
masked q.k^T block and dv_local itself; every stored dh snapshot and the
bf16(dh) fed to k.dh; dv2; the products w^T bf16(dv2) and q e^{g} (fp32,
the reference's promoted operand) times do; ds; dq, dk, -dw; the WY terms
bf16(k beta e^{g}), bf16(v beta), bf16(k beta), bf16(dA) (twice) and the
stored dk / dv; dk + dk2 added in bf16; dg in fp32.  "fp32" and "fp64" modes
have no rounding points; "fp64" is exact algebra.

Pinned by tests/test_oracle_bwd.py: in fp64 every gradient (dq, dk, dv, dg,
dbeta, dh0, with and without the in-kernel L2 norm, ragged tails, varlen,
initial and final-state gradients) equals torch autograd of the fp64 token
recurrence to < 1e-9; that autograd is itself checked by central finite
differences of ``gdn_oracle.naive_recurrent``; and planted mistakes (a
missing reverse cumsum, a dropped WY term, a wrong dh decay, an unmasked
diagonal in dv_local) each fail the autograd check.
"""
from __future__ import annotations

import numpy as np

from . import gdn_oracle as O

__all__ = ["chunk_gated_delta_rule_bwd", "l2norm_fwd_rstd", "l2norm_bwd", "reverse_chunk_cumsum"]


def _T(x):
    return np.ascontiguousarray(np.swapaxes(x, -1, -2))


def l2norm_fwd_rstd(x, eps: float = 1e-6, dtype: str = "fp32"):
    """(y, rstd): y = x rstd in the storage dtype, rstd = 1 / sqrt(sum x^2 + eps) fp32 (l2norm.py:98-130)."""
    f = O._f(dtype)
    xf = np.asarray(x, f)
    rstd = 1.0 / np.sqrt(np.sum(xf * xf, axis=-1, keepdims=True) + eps)
    return O.cast(xf * rstd, dtype), rstd[..., 0]


def l2norm_bwd(y, rstd, dy, dtype: str = "fp32"):
    """dx = dy rstd - sum(dy y) y rstd per row, stored in y's dtype (l2norm.py:132-154)."""
    f = O._f(dtype)
    yf, dyf = np.asarray(y, f), np.asarray(dy, f)
    r = np.asarray(rstd, f)[..., None]
    return O.cast(dyf * r - np.sum(dyf * yf, axis=-1, keepdims=True) * yf * r, dtype)


def reverse_chunk_cumsum(dgc, cm: O.ChunkMap):
    """Suffix sums within each chunk over the valid rows (cumsum.py:58-63 with REVERSE): [NC, H, C]."""
    d = np.where(cm.valid[:, None, :], dgc, 0.0)
    return np.flip(np.cumsum(np.flip(d, axis=-1), axis=-1), axis=-1)


def _dv_local_c(cm, qc, kc, doc, gcc, scale, f, dtype):
    """chunk_o.py:413-468: dv_local = mask_{j<=i}(scale k_j.q_i e^{g_i - g_j}) (stored) @ do."""
    m = np.swapaxes(O._pair_mask(cm, False), -1, -2)              # [NC, 1, j, i]: j <= i, both valid
    At = (kc @ _T(qc)) * scale                                   # [NC, H, j, i]
    At = At * np.exp(np.where(m, gcc[..., None, :] - gcc[..., :, None], 0.0))
    At = O.cast(np.where(m, At, 0.0), dtype)
    return O.cast(At @ doc, dtype)


def _dhu_c(cm, qc, kc, wc, doc, dvc, gcc, scale, h0, dht, f, dtype):
    """chunk_delta_h.py:250-438: reverse recurrence of dh; returns (dh snapshots [NC,H,K,V], dh0, dv2 [NC,H,C,V])."""
    NC, H, C, K = kc.shape
    V = doc.shape[-1]
    dh_snap = np.zeros((NC, H, K, V), f)
    dv2 = np.zeros((NC, H, C, V), f)
    dh0 = np.zeros((len(cm.spans), H, K, V), f) if h0 is not None else None
    for n in range(len(cm.spans)):
        dh = np.zeros((H, K, V), f)
        if dht is not None:
            dh = dh + np.asarray(dht[n], f)
        for c in range(cm.chunk_offsets[n + 1] - 1, cm.chunk_offsets[n] - 1, -1):
            dhs = O.cast(dh, dtype)
            dh_snap[c] = dhs
            valid = cm.valid[c][None, :]                            # [1, C]
            g_last = gcc[c, :, cm.nv[c] - 1]                        # [H]
            gate = np.where(valid, np.exp(g_last[:, None] - gcc[c]), 0.0)
            dv = (kc[c] @ dhs) * gate[..., None] + dvc[c]           # [H, C, V]
            dv2[c] = O.cast(dv, dtype)
            qg = qc[c] * np.exp(np.where(valid, gcc[c], 0.0))[..., None]
            dh = dh * np.exp(g_last)[:, None, None] + (_T(qg) @ doc[c]) * scale - _T(wc[c]) @ dv2[c]
        if dh0 is not None:
            dh0[n] = dh
    return dh_snap, dh0, dv2


def _dqkwg_c(cm, qc, kc, vnc, doc, h, dh, dv2, gcc, scale, f, dtype):
    """chunk_o.py:147-326 with USE_G and USE_DW: (dq, dk, dw, dg) per chunk."""
    valid = cm.valid[:, None, :]                                   # [NC, 1, C]
    ds = doc @ _T(vnc)                                             # [NC, H, C, C]
    dq = doc @ _T(h)                                               # [NC, H, C, K]
    dk = vnc @ _T(dh)
    dw = O.cast(-(dv2 @ _T(h)), dtype)
    dg_last = np.sum(h * dh, axis=(-1, -2))                        # [NC, H]
    g_last = np.take_along_axis(gcc, (cm.nv - 1)[:, None, None].repeat(gcc.shape[1], 1), axis=2)[..., 0]
    dg_last = dg_last * np.exp(g_last)
    dq = dq * np.exp(gcc)[..., None] * scale
    dg = np.sum(dq * qc, axis=-1)
    dk = dk * np.where(valid, np.exp(g_last[..., None] - gcc), 0.0)[..., None]
    dg = dg - np.sum(kc * dk, axis=-1)
    dg_last = dg_last + np.sum(dk * kc, axis=(-1, -2))
    m = O._pair_mask(cm, False)                                    # i >= j, both valid
    ds = np.where(m, ds * np.exp(np.where(m, gcc[..., :, None] - gcc[..., None, :], 0.0)), 0.0) * scale
    ds2 = ds * (qc @ _T(kc))
    dg = dg + np.sum(ds2, axis=-1) - np.sum(ds2, axis=-2)
    ds = O.cast(ds, dtype)
    dq = dq + ds @ kc
    dk = dk + _T(ds) @ qc
    last = np.zeros_like(cm.valid)
    last[np.arange(cm.nc), cm.nv - 1] = True
    dg = dg + np.where(last[:, None, :], dg_last[..., None], 0.0)
    return O.cast(dq, dtype), O.cast(dk, dtype), dw, dg


def _wy_bwd_c(cm, kc, vc, bc, Aic, gcc, dwc, duc, f, dtype):
    """wy_fast.py:98-210 with USE_G: (dk2, dv, db, dg2) per chunk."""
    AiT = _T(Aic)                                                  # the reference loads A transposed
    eg = np.exp(gcc)
    kbg = kc * (bc * eg)[..., None]
    dA = dwc @ _T(O.cast(kbg, dtype))
    dkbg = AiT @ dwc
    dk = O.cast(dkbg * (eg * bc)[..., None], dtype)
    db = np.sum(dkbg * kc * eg[..., None], axis=-1)
    dg = np.sum(dkbg * kbg, axis=-1)
    vb = O.cast(vc * bc[..., None], dtype)
    dA = dA + duc @ _T(vb)
    dvb = AiT @ duc
    dv = O.cast(dvb * bc[..., None], dtype)
    db = db + np.sum(dvb * vc, axis=-1)
    strict = O._pair_mask(cm, True)
    dA = np.where(strict, dA, 0.0)
    dA = O.cast(dA, dtype) @ AiT
    dA = AiT @ O.cast(dA, dtype)
    dA = dA * np.exp(np.where(strict, gcc[..., :, None] - gcc[..., None, :], 0.0))
    dA = O.cast(np.where(strict, -dA, 0.0), dtype)
    kb = O.cast(kc * bc[..., None], dtype)
    A2 = kb @ _T(kc)
    dkb = dA @ kc
    db = db + np.sum(dkb * kc, axis=-1)
    dk = O.cast(dk + _T(dA) @ kb + dkb * bc[..., None], dtype)
    AdA = dA * A2
    dg = dg + np.sum(AdA, axis=-1) - np.sum(AdA, axis=-2)
    return dk, dv, db, dg


def chunk_gated_delta_rule_bwd(q, k, v, g, beta, do, dht=None, scale=None, initial_state=None,
                               use_qk_l2norm_in_kernel=False, cu_seqlens=None, dtype: str = "fp32",
                               beta_dtype: str | None = None, return_intermediates: bool = False):
    """Gradients of chunk_gated_delta_rule (chunk.py:188-213 -> :70-146) for o-gradient ``do`` and
    final-state gradient ``dht`` (None = zero).  Inputs hold values representable in ``dtype`` (q, k, v,
    beta, do) and fp32 g.  Returns (dq, dk, dv, dg, dbeta, dh0); dh0 is None without an initial state.
    """
    B, T, H, K = q.shape
    if scale is None:
        scale = K ** -0.5
    f = O._f(dtype)
    bdt = beta_dtype or dtype
    q_in, k_in = q, k
    if use_qk_l2norm_in_kernel:
        q, q_rstd = l2norm_fwd_rstd(q_in, dtype=dtype)
        k, k_rstd = l2norm_fwd_rstd(k_in, dtype=dtype)
    cm = O.ChunkMap(B, T, cu_seqlens, O.CHUNK)
    qc, kc, vc = cm.gather(q, f), cm.gather(k, f), cm.gather(v, f)
    bc, doc = cm.gather(beta, f), cm.gather(do, f)
    gcc = O._cumsum_c(cm.gather(g, f), f)
    # forward recomputation (chunk.py:84-101): Ai from the forward, then w, u, h, v_new
    Ac = O._kkt_c(cm, kc, gcc, bc, f)
    Aic = O.cast(O._solve_c(Ac, f), dtype)
    wc, uc = O._wu_c(kc, vc, bc, Aic, gcc, f, dtype)
    h, vnc, _ = O._fwd_h_c(cm, kc, wc, uc, gcc, initial_state, f, dtype)
    dvl = _dv_local_c(cm, qc, kc, doc, gcc, scale, f, dtype)
    dh, dh0, dv2 = _dhu_c(cm, qc, kc, wc, doc, dvl, gcc, scale, initial_state, dht, f, dtype)
    dq, dk, dw, dg = _dqkwg_c(cm, qc, kc, vnc, doc, h, dh, dv2, gcc, scale, f, dtype)
    dk2, dv, db, dg2 = _wy_bwd_c(cm, kc, vc, bc, Aic, gcc, dw, dv2, f, dtype)
    dk = O.cast(dk + dk2, dtype)
    dgc = reverse_chunk_cumsum(dg + dg2, cm)
    dq_t, dk_t = cm.scatter(dq, f), cm.scatter(dk, f)
    if use_qk_l2norm_in_kernel:
        dq_t = l2norm_bwd(q, q_rstd, dq_t, dtype)
        dk_t = l2norm_bwd(k, k_rstd, dk_t, dtype)
    out = (dq_t, dk_t, cm.scatter(dv, f), cm.scatter(dgc, f), O.cast(cm.scatter(db, f), bdt), dh0)
    if return_intermediates:
        inter = dict(dv_local=cm.scatter(dvl, f), dh=dh, dv2=cm.scatter(dv2, f), dw=cm.scatter(dw, f),
                     dq=cm.scatter(dq, f), dk=cm.scatter(dk, f), dk2=cm.scatter(dk2, f), dg_pre=cm.scatter(dg, f),
                     dg2_pre=cm.scatter(dg2, f), h=h, v_new=cm.scatter(vnc, f), w=cm.scatter(wc, f),
                     Ai=cm.scatter(Aic, f), gc=cm.scatter(gcc, f))
        return out, inter
    return out
