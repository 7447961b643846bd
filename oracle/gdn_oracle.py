"""CPU restatement of the chunked GatedDeltaNet forward -- TEST INFRASTRUCTURE ONLY.

This module is the parity oracle for the HIP kernels in ``kairos-sensenova_amd``.
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and only as the checker; the product path never calls it.

It restates, stage by stage, the reference op
``chunk_gated_delta_rule`` of flash-linear-attention 0.4.0 as vendored in
``kairos/third_party/fla`` (paths below are relative to that tree):

  stage                      reference
  -------------------------  ------------------------------------------------
  l2norm                     modules/l2norm.py:114-118 (eps 1e-6, :159)
  chunk_local_cumsum         ops/utils/cumsum.py:27-65, :247-279
  chunk_scaled_dot_kkt       ops/common/chunk_scaled_dot_kkt.py:57-73
  solve_tril                 ops/utils/solve_tril.py:184-331 ((I+A)^-1, RTNE out)
  recompute_w_u              ops/gated_delta_rule/wy_fast.py:55-81
  chunk_fwd_h                ops/common/chunk_delta_h.py:113-224
  chunk_fwd_o                ops/common/chunk_o.py:84-128
  chunk_gated_delta_rule     ops/gated_delta_rule/chunk.py:16-67, :149-186, :217-323
  naive_recurrent            ops/gated_delta_product/naive.py:23-35 (num_householder=1),
                             ops/gated_delta_rule/fused_recurrent.py:88-119
  fused_recurrent            ops/gated_delta_rule/fused_recurrent.py:21-135, :238-349
                             (gk / gv decays, per-column beta, grouped value heads)
  causal_conv1d              modules/convolution.py:54-141, :410-458, :539-602 (the
                             layer's ShortConvolution with SiLU, cache in / out)
  gdn_gates                  layers/gated_deltanet.py:265-271
  rms_norm_gated             modules/fused_norm_gate.py:42-127 (RMS path, no residual),
                             the layer's output epilogue (layers/gated_deltanet.py:197,311)

Precision model (``dtype`` argument):
  "bf16"  storage values are bf16 held in float32 arrays; every cast point of
          the reference (Ai, w, u, h snapshot, v_new, Aqk, o, and the
          bf16*bf16 products of Triton's type promotion) is rounded to bf16
          with round-to-nearest-even; dots accumulate in float32.
  "fp32"  all storage and arithmetic in float32 (no rounding points).
  "fp64"  all storage and arithmetic in float64: the exact-algebra mode used
          to pin the chunked form against the token recurrence.

How each function is pinned (tests/test_oracle.py):
  chunk_local_cumsum     closed form: per-chunk numpy cumsum restarting at chunk
                         and sequence starts; varlen == separate sequences.
  chunk_scaled_dot_kkt   brute-force per-element loop on tiny inputs.
  solve_tril             numpy.linalg.inv(I + A) and (I + A) @ Ai == I.
  recompute_w_u          chunk algebra: with h = 0, v_new of the first chunk
                         equals u and the state recurrence pins w (below).
  chunk_fwd_h / fwd_o /  fp64 chunked result == fp64 token recurrence
  chunk_gated_delta_rule (<1e-10), plus invariants (beta=0 decay, g->-inf
                         reset, chunk-size independence 16/32/64, split calls
                         with state carry, varlen == separate calls, linearity
                         in (v, h0), causality of padded tails) and planted
                         mistakes (I-A solve sign, decayed v_new, strict output
                         mask, missing beta, non-restarting cumsum) that each
                         fail the recurrence check.
  naive_recurrent        closed forms: beta=0 pure decay; beta=1, g=0, unit k
                         gives exact recall S^T k_t = v_t; a hand-computed
                         two-token case.
  fused_recurrent        == naive_recurrent (fp64) for scalar gates and per-head
                         beta; gk (resp. gv) equal to g broadcast over K (V)
                         == the g path; beta = 0 closed forms S_T = diag(e^{sum gk})
                         h0 and h0 diag(e^{sum gv}); per-column beta of equal
                         columns == per-head beta, one-token closed form
                         S = k (beta v)^T; grouped value heads == q/k repeated;
                         in-kernel L2 norm == normalised inputs; planted
                         mistakes (gk applied over V, decay after the delta,
                         wrong q/k head for a value head) each fail one check.
  causal_conv1d          torch.nn.functional.conv1d (fp64, groups=D, causal
                         padding) without a cache; split calls with the cache
                         carried == one call; final state == last W of [cache, x];
                         varlen == separate calls; planted reversed taps fail.
  gdn_gates              torch softplus / sigmoid / exp (fp64) and the closed
                         form a + dt_bias = 0 -> g = -exp(A_log) log 2.
  l2norm                 closed form x / sqrt(sum x^2 + eps).
  rms_norm_gated         torch.nn.functional.rms_norm times silu / sigmoid of the
                         gate (library routines, fp64); closed forms: g = 0 gives
                         0 (swish) or half the normalised row (sigmoid), a
                         constant row normalises to sign * |c| / sqrt(c^2 + eps),
                         scaling x leaves y unchanged when eps = 0.
Every function above has at least one such check: no function is left
"parity unpinned".
"""
from __future__ import annotations

import math

import numpy as np

CHUNK = 64

__all__ = [
    "CHUNK", "to_bf16", "cast", "seq_spans", "l2norm", "chunk_local_cumsum",
    "chunk_scaled_dot_kkt", "solve_tril", "recompute_w_u", "chunk_fwd_h",
    "chunk_fwd_o", "chunk_gated_delta_rule", "naive_recurrent", "rel_l2",
    "fp8_e4m3_quantize", "fp8_e4m3_decode", "rms_norm_gated", "fused_recurrent", "causal_conv1d", "gdn_gates",
]


# ----------------------------------------------------------------------------
# rounding helpers
# ----------------------------------------------------------------------------
def to_bf16(x) -> np.ndarray:
    """Round float32 values to bf16 with round-to-nearest-even; returns float32."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32)
    r = (u >> np.uint32(16)) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32).reshape(a.shape)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def _ftype(dtype: str):
    return np.float64 if dtype == "fp64" else np.float32


def cast(x, dtype: str) -> np.ndarray:
    """Round ``x`` to the storage precision named by ``dtype``."""
    if dtype == "bf16":
        return to_bf16(x)
    return np.asarray(x, dtype=_ftype(dtype))


def _mul_store(a, b, dtype: str) -> np.ndarray:
    """Elementwise product in the storage dtype.

    Triton promotes bf16*bf16 to bf16 (the product is formed in fp32 and
    rounded), which is what wy_fast.py:65,77 do when beta is bf16.
    """
    return cast(np.asarray(a, _ftype(dtype)) * np.asarray(b, _ftype(dtype)), dtype)


def rel_l2(x, ref) -> float:
    """RMS(x - ref) / RMS(ref): fla's get_err_ratio (fla/utils.py:76-79)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    err = math.sqrt(float(np.mean(np.square(x - ref)))) if x.size else 0.0
    base = math.sqrt(float(np.mean(np.square(ref)))) if ref.size else 0.0
    return err / (base + 1e-8)


# ----------------------------------------------------------------------------
# fp8 e4m3 (OCP "fn" variant, as torch.float8_e4m3fn): used by the streaming config
# ----------------------------------------------------------------------------
def fp8_e4m3_decode(codes) -> np.ndarray:
    """Decode uint8 e4m3fn codes to float32 (exact)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = (c & 0x7).astype(np.float64)
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((e == 15) & ((c & 7) == 7), np.nan, val)
    return (s * val).astype(np.float32)


_E4M3_TABLE = fp8_e4m3_decode(np.arange(256, dtype=np.uint8))


def fp8_e4m3_quantize(x) -> np.ndarray:
    """Round float values to the nearest e4m3fn code (ties to even code), saturating at 448."""
    x = np.clip(np.asarray(x, np.float64), -448.0, 448.0)
    pos = _E4M3_TABLE[:127].astype(np.float64)            # codes 0..126 are the finite non-negatives
    mag = np.abs(x)
    idx = np.searchsorted(pos, mag)                        # pos[idx-1] < mag <= pos[idx]
    idx = np.clip(idx, 1, 126)
    lo, hi = pos[idx - 1], pos[idx]
    pick_hi = (mag - lo > hi - mag) | ((mag - lo == hi - mag) & ((idx % 2) == 0))
    code = np.where(pick_hi, idx, idx - 1).astype(np.uint8)
    code = np.where(mag == 0, 0, code).astype(np.uint8)
    return np.where(x < 0, code | 0x80, code).astype(np.uint8)


# ----------------------------------------------------------------------------
# sequence / chunk bookkeeping (fla/ops/utils/index.py:113-127)
# ----------------------------------------------------------------------------
def seq_spans(B: int, T: int, cu_seqlens=None):
    """List of (batch_row, bos, eos) for every sequence.

    Fixed length: one sequence per batch row.  Varlen (B must be 1): the
    sequences are the slices of ``cu_seqlens`` (index.py:113-119).
    """
    if cu_seqlens is None:
        return [(b, 0, T) for b in range(B)]
    cu = [int(x) for x in np.asarray(cu_seqlens).tolist()]
    return [(0, cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


class ChunkMap:
    """Token index of every (chunk, row) slot, chunks of all sequences in order.

    Mirrors prepare_chunk_indices / prepare_chunk_offsets (index.py:113-127):
    chunks restart at every sequence start, the last chunk of a sequence may be
    ragged.  ``idx`` points into the flattened [B*T] token axis; padded slots
    point at an extra all-zero row (index B*T) and have ``valid`` False.
    Chunked arrays use the layout [NC, H, C, ...] (heads before rows).
    """

    def __init__(self, B: int, T: int, cu_seqlens=None, chunk: int = CHUNK):
        self.B, self.T, self.chunk = B, T, chunk
        self.spans = seq_spans(B, T, cu_seqlens)
        idx, self.chunk_offsets = [], [0]
        for b, bos, eos in self.spans:
            for t0 in range(bos, eos, chunk):
                rows = np.arange(t0, t0 + chunk)
                idx.append(np.where(rows < eos, b * T + rows, B * T))
            self.chunk_offsets.append(len(idx))
        self.idx = np.array(idx, dtype=np.int64).reshape(-1, chunk)
        self.valid = self.idx < B * T
        self.nv = self.valid.sum(axis=1)
        self.nc = self.idx.shape[0]
        self.dense = cu_seqlens is None and T % chunk == 0

    def gather(self, x, f):
        """[B, T, H, ...] -> contiguous [NC, H, C, ...] with zeros in padded slots."""
        x = np.asarray(x)
        rest = x.shape[3:]
        H = x.shape[2]
        if self.dense:
            xc = x.reshape(self.nc, self.chunk, H, *rest)
        else:
            flat = x.reshape(self.B * self.T, H, *rest)
            flat = np.concatenate([flat, np.zeros((1, H) + rest, flat.dtype)], axis=0)
            xc = flat[self.idx]
        return np.ascontiguousarray(np.moveaxis(xc, 2, 1), dtype=f)

    def scatter(self, xc, f):
        """contiguous [NC, H, C, ...] -> [B, T, H, ...] (padded slots dropped)."""
        xt = np.ascontiguousarray(np.moveaxis(xc, 1, 2), dtype=f)          # [NC, C, H, ...]
        if self.dense:
            return xt.reshape(self.B, self.T, *xt.shape[2:])
        out = np.zeros((self.B * self.T + 1,) + xt.shape[2:], f)
        out[self.idx[self.valid]] = xt[self.valid]
        return out[:-1].reshape(self.B, self.T, *xt.shape[2:])


def _f(dtype):
    return np.float64 if dtype == "fp64" else np.float32


def _lower(C, strict):
    return np.tril(np.ones((C, C), bool), -1 if strict else 0)


def _pair_mask(cm: ChunkMap, strict: bool):
    """[NC, 1, C, C]: lower-triangular (strict or with diagonal) over valid rows and columns."""
    v = cm.valid
    return (_lower(cm.chunk, strict)[None] & v[:, :, None] & v[:, None, :])[:, None]


# ----------------------------------------------------------------------------
# stages on chunked arrays ([NC, H, C, ...]); the public wrappers follow
# ----------------------------------------------------------------------------
def _cumsum_c(gc_in, f):
    return np.cumsum(gc_in, axis=2, dtype=f)                   # padded slots hold 0


def _kkt_c(cm, kc, gcc, bc, f):
    dots = kc @ np.ascontiguousarray(np.swapaxes(kc, 2, 3))    # [NC, H, C, C]
    m = _pair_mask(cm, True)
    diff = np.where(m, gcc[..., :, None] - gcc[..., None, :], 0.0)
    return np.where(m, dots * np.exp(diff) * bc[..., :, None], 0.0).astype(f)


def _solve_c(Ac, f):
    C = Ac.shape[-1]
    X = np.zeros_like(Ac, dtype=f)
    L = np.asarray(Ac, f)
    for i in range(C):
        # x_i = e_i - sum_{r<i} L[i, r] x_r   (rows of the inverse, unit diagonal)
        if i:
            X[:, :, i, :] = -np.einsum("nhr,nhrc->nhc", L[:, :, i, :i], X[:, :, :i, :])
        X[:, :, i, i] = 1.0
    return X


def _wu_c(kc, vc, bc, Aic, gcc, f, dtype):
    bet = bc[..., None]
    vb = _mul_store(vc, bet, dtype)
    kb = _mul_store(kc, bet, dtype)
    kb = cast(kb * np.exp(gcc)[..., None], dtype)
    return cast(Aic @ kb, dtype), cast(Aic @ vb, dtype)


def _fwd_h_c(cm, kc, wc, uc, gcc, initial_state, f, dtype):
    NC, H, C, K = kc.shape
    V = uc.shape[-1]
    kT = np.ascontiguousarray(np.swapaxes(kc, 2, 3))              # [NC, H, K, C]
    h = np.zeros((NC, H, K, V), f)
    vnew = np.zeros((NC, H, C, V), f)
    ht = np.zeros((len(cm.spans), H, K, V), f)
    for n in range(len(cm.spans)):
        S = np.zeros((H, K, V), f)
        if initial_state is not None:
            S = S + np.asarray(initial_state[n], f)
        for c in range(cm.chunk_offsets[n], cm.chunk_offsets[n + 1]):
            hc = cast(S, dtype)
            h[c] = hc
            vp = uc[c] - wc[c] @ hc                                 # [H, C, V]
            vnew[c] = cast(vp, dtype)
            g_last = gcc[c, :, cm.nv[c] - 1]                        # [H]
            gate = np.where(cm.valid[c][None, :], np.exp(g_last[:, None] - gcc[c]), 0.0)
            S = S * np.exp(g_last)[:, None, None]
            S = S + kT[c] @ cast(vp * gate[:, :, None], dtype)
        ht[n] = S
    return h, vnew, ht


def _fwd_o_c(cm, qc, kc, vnc, h, gcc, scale, f, dtype):
    o1 = (qc @ np.asarray(h, f)) * np.exp(gcc)[..., None]
    m = _pair_mask(cm, False)
    diff = np.where(m, gcc[..., :, None] - gcc[..., None, :], 0.0)
    Aqk = np.where(m, (qc @ np.ascontiguousarray(np.swapaxes(kc, 2, 3))) * np.exp(diff), 0.0).astype(f)
    return cast(o1 * scale + (cast(Aqk, dtype) @ vnc) * scale, dtype)


# ----------------------------------------------------------------------------
# public stages ([B, T, H, ...] layout, as the reference's stage functions)
# ----------------------------------------------------------------------------
def rms_norm_gated(x, g, weight=None, bias=None, activation: str = "swish", eps: float = 1e-6,
                   dtype: str = "fp32"):
    """Gated RMSNorm over the last axis (fused_norm_gate.py:42-127 with
    IS_RMS_NORM, no residual): x and g upcast, rstd = 1/sqrt(mean(x^2) + eps)
    (:83-89), y = x rstd [* w] [+ b] (:94-100), then y * g * sigmoid(g) for
    'swish'/'silu' or y * sigmoid(g) for 'sigmoid' (:102-108); y stored in
    ``dtype`` (the input's storage dtype).  Returns (y, rstd)."""
    f = _f(dtype)
    xf = np.asarray(x, f)
    gf = np.asarray(g, f)
    rstd = (1.0 / np.sqrt(np.mean(xf * xf, axis=-1) + eps)).astype(f)
    y = xf * rstd[..., None]
    if weight is not None:
        y = y * np.asarray(weight, f)
    if bias is not None:
        y = y + np.asarray(bias, f)
    sig = 1.0 / (1.0 + np.exp(-gf))
    if activation in ("swish", "silu"):
        y = y * gf * sig
    elif activation == "sigmoid":
        y = y * sig
    else:
        raise ValueError(f"Unsupported activation: {activation}")
    return cast(y, dtype), rstd


def l2norm(x, eps: float = 1e-6, dtype: str = "fp32") -> np.ndarray:
    """y = x / sqrt(sum(x^2) + eps) along the last axis (l2norm.py:114-118), stored in ``dtype``."""
    xf = np.asarray(x, _f(dtype))
    rstd = 1.0 / np.sqrt(np.sum(xf * xf, axis=-1, keepdims=True) + eps)
    return cast(xf * rstd, dtype)


def chunk_local_cumsum(g, cu_seqlens=None, chunk: int = CHUNK, dtype: str = "fp32") -> np.ndarray:
    """Prefix sum of g inside each chunk, restarting at chunk and sequence starts.

    cumsum.py:58-59 (fp32 load and tl.cumsum), output fp32 (:254, :264).
    """
    B, T, H = g.shape
    f = _f(dtype)
    cm = ChunkMap(B, T, cu_seqlens, chunk)
    return cm.scatter(_cumsum_c(cm.gather(g, f), f), f)


def chunk_scaled_dot_kkt(k, gc, beta, cu_seqlens=None, chunk: int = CHUNK, dtype: str = "fp32") -> np.ndarray:
    """A[t, h, j] = beta_i * exp(gc_i - gc_j) * (k_i . k_j) for i > j inside the chunk, else 0.

    chunk_scaled_dot_kkt.py:57-73: fp32 dot of the stored k, then * exp(g_i - g_j),
    then * beta_i, strictly-lower mask over valid rows; stored fp32 as [B, T, H, BT].
    """
    B, T, H, K = k.shape
    f = _f(dtype)
    cm = ChunkMap(B, T, cu_seqlens, chunk)
    return cm.scatter(_kkt_c(cm, cm.gather(k, f), cm.gather(gc, f), cm.gather(beta, f), f), f)


def solve_tril(A, cu_seqlens=None, chunk: int = CHUNK, dtype: str = "fp32") -> np.ndarray:
    """Ai = (I + A)^-1 per chunk (A strictly lower), computed in fp32, stored in ``dtype`` (RTNE).

    solve_tril.py:184-331 inverts the 16x16 diagonal blocks by forward
    substitution and merges them in fp32 ('ieee' dots, :13), then stores with
    fp_downcast_rounding='rtne' (:311-320).  Here: forward substitution of the
    whole chunk in the working precision (same mathematics).  Padded rows of a
    ragged chunk get the identity row, which only meets zero columns of A.
    """
    B, T, H, C = A.shape
    f = _f(dtype)
    cm = ChunkMap(B, T, cu_seqlens, C)
    return cast(cm.scatter(_solve_c(cm.gather(A, f), f), f), dtype)


def recompute_w_u(k, v, beta, Ai, gc, cu_seqlens=None, chunk: int = CHUNK, dtype: str = "fp32"):
    """u = Ai @ (v * beta), w = Ai @ (k * beta * exp(gc)); both stored in the k/v dtype.

    wy_fast.py:55-81: vb = (v * beta).to(v.dtype) (:65); kb = k * beta (:77),
    kb *= exp(g) (:79), cast to k.dtype (:80); dots accumulate in fp32.
    """
    B, T, H, K = k.shape
    f = _f(dtype)
    cm = ChunkMap(B, T, cu_seqlens, chunk)
    wc, uc = _wu_c(cm.gather(k, f), cm.gather(v, f), cm.gather(beta, f), cm.gather(Ai, f),
                   cm.gather(gc, f), f, dtype)
    return cm.scatter(wc, f), cm.scatter(uc, f)


def chunk_fwd_h(k, w, u, gc, initial_state=None, output_final_state=False, cu_seqlens=None,
                chunk: int = CHUNK, dtype: str = "fp32"):
    """Serial inter-chunk state recurrence (chunk_delta_h.py:113-224).

    For each sequence and chunk c, with S the fp32 state [H, K, V]:
      h[c]  = S stored in k.dtype                          (:129-139)
      v'    = u_c - w_c @ h[c]   (dot with the *stored* h)  (:141-157)
      v_new = v' stored ungated in u.dtype                  (:159-161)
      v'   *= exp(g_last - g) for valid rows, 0 otherwise   (:163-169)
      S    *= exp(g_last)                                    (:170-177)
      S    += k_c^T @ v'.to(k.dtype)                          (:195-211)
    ht = S after the last chunk, fp32 (:213-224).
    Returns h [NT_total, H, K, V] (chunks of all sequences in order), v_new
    [B, T, H, V] and ht [N, H, K, V] (or None).
    """
    B, T, H, K = k.shape
    f = _f(dtype)
    cm = ChunkMap(B, T, cu_seqlens, chunk)
    h, vnew, ht = _fwd_h_c(cm, cm.gather(k, f), cm.gather(w, f), cm.gather(u, f), cm.gather(gc, f),
                           initial_state, f, dtype)
    return h, cm.scatter(vnew, f), (ht if output_final_state else None)


def chunk_fwd_o(q, k, v_new, h, gc, scale, cu_seqlens=None, chunk: int = CHUNK, dtype: str = "fp32"):
    """o = scale * (q @ h_c) * exp(gc) + scale * (mask_{i>=j}(q k^T * exp(gc_i - gc_j))).to(v) @ v_new.

    chunk_o.py:84-128: both dots accumulate in fp32 over the stored operands;
    the causal mask includes the diagonal (:118); the attention block is cast
    to v's dtype before its dot (:127); o is stored in v's dtype (:516).
    """
    B, T, H, K = q.shape
    f = _f(dtype)
    cm = ChunkMap(B, T, cu_seqlens, chunk)
    oc = _fwd_o_c(cm, cm.gather(q, f), cm.gather(k, f), cm.gather(v_new, f), h, cm.gather(gc, f),
                  scale, f, dtype)
    return cm.scatter(oc, f)


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                           use_qk_l2norm_in_kernel=False, cu_seqlens=None, chunk: int = CHUNK,
                           dtype: str = "fp32", return_intermediates: bool = False):
    """Whole forward: chunk.py:217-323 (entry, scale default, varlen checks),
    :149-186 (optional q/k L2 norm), :16-67 (stage order).  Inputs must already
    hold values representable in ``dtype`` (q, k, v, beta) and fp32 g.
    Returns (o, final_state) in the storage dtype / fp32.
    """
    B, T, H, K = q.shape
    if cu_seqlens is not None:
        if B != 1:
            raise ValueError("The batch size is expected to be 1 when using `cu_seqlens`.")
        if initial_state is not None and initial_state.shape[0] != len(cu_seqlens) - 1:
            raise ValueError("The number of initial states is expected to be equal to the number of input sequences")
    if scale is None:
        scale = K ** -0.5
    if use_qk_l2norm_in_kernel:
        q = l2norm(q, dtype=dtype)
        k = l2norm(k, dtype=dtype)
    f = _f(dtype)
    cm = ChunkMap(B, T, cu_seqlens, chunk)
    qc, kc, vc = cm.gather(q, f), cm.gather(k, f), cm.gather(v, f)
    bc = cm.gather(beta, f)
    gcc = _cumsum_c(cm.gather(g, f), f)
    Ac = _kkt_c(cm, kc, gcc, bc, f)
    Aic = cast(_solve_c(Ac, f), dtype)
    wc, uc = _wu_c(kc, vc, bc, Aic, gcc, f, dtype)
    h, vnc, ht = _fwd_h_c(cm, kc, wc, uc, gcc, initial_state, f, dtype)
    o = cm.scatter(_fwd_o_c(cm, qc, kc, vnc, h, gcc, scale, f, dtype), f)
    ht = ht if output_final_state else None
    if return_intermediates:
        inter = dict(gc=cm.scatter(gcc, f), A=cm.scatter(Ac, f), Ai=cm.scatter(Aic, f),
                     w=cm.scatter(wc, f), u=cm.scatter(uc, f), h=h, v_new=cm.scatter(vnc, f), q=q, k=k)
        return o, ht, inter
    return o, ht


def _rec_heads(x, rep):
    """q/k heads -> value heads: head h serves value heads h*rep .. h*rep+rep-1 (fused_recurrent.py:53)."""
    return np.repeat(x, rep, axis=2)


def _rec_decay(f, g_t, gk_t, gv_t, HV, K, V):
    """Multiplicative decay of the [HV, K, V] state for one token (fused_recurrent.py:104-114)."""
    d = np.ones((HV, K, V), f)
    if g_t is not None:
        d = d * np.exp(np.asarray(g_t, f))[:, None, None]
    if gk_t is not None:
        d = d * np.exp(np.asarray(gk_t, f))[:, :, None]
    if gv_t is not None:
        d = d * np.exp(np.asarray(gv_t, f))[:, None, :]
    return d


def _rec_token(S, decay, qt, kt, vt, bt):
    """One token: decay, delta-rule write, read (fused_recurrent.py:104-122).  Returns (S, o_t)."""
    S = S * decay
    vp = bt * (vt - np.sum(S * kt[:, :, None], axis=1))
    S = S + kt[:, :, None] * vp[:, None, :]
    return S, np.sum(S * qt[:, :, None], axis=1)


def fused_recurrent(q, k, v, g=None, gk=None, gv=None, beta=None, scale=None, initial_state=None, cu_seqlens=None,
                    use_qk_l2norm_in_kernel=False, dtype: str = "fp32", o_dtype: str = "fp32"):
    """The short-sequence mode fused_recurrent_gated_delta_rule (fused_recurrent.py:21-135, :238-349),
    restated per token in ``dtype`` arithmetic ("fp32" as the kernel, or "fp64"):

        q, k <- [l2-normalised];  q <- q * scale
        S <- S * exp(g) * exp(gk)[:, None] * exp(gv)[None, :]     (each decay optional)
        v' = beta * (v - S^T k)                                    (beta per head or per column)
        S <- S + k v'^T ;  o = S^T q   (o rounded to ``o_dtype``, v's storage dtype)
    Shapes: q, k [B, T, H, K]; v [B, T, HV, V], HV a multiple of H, q/k head
    hv // (HV // H) serving value head hv (fused_recurrent.py:53); g [B, T, HV];
    gk [B, T, HV, K]; gv [B, T, HV, V]; beta [B, T, HV] or [B, T, HV, V] (None:
    ones).  Returns (o [B, T, HV, V], ht [N, HV, K, V]) as float32 (float64 for "fp64").
    """
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    f = np.float64 if dtype == "fp64" else np.float32
    if scale is None:
        scale = K ** -0.5
    qf = _rec_heads(np.asarray(q, f), HV // H)              # [B, T, HV, K]
    kf = _rec_heads(np.asarray(k, f), HV // H)
    vf = np.asarray(v, f)
    if use_qk_l2norm_in_kernel:
        qf = qf / np.sqrt(np.sum(qf * qf, axis=-1, keepdims=True) + f(1e-6))
        kf = kf / np.sqrt(np.sum(kf * kf, axis=-1, keepdims=True) + f(1e-6))
    qf = qf * f(scale)
    if beta is None:
        bf = np.ones((B, T, HV, 1), f)
    else:
        bf = np.asarray(beta, f)
        bf = bf[..., None] if bf.ndim == 3 else bf            # [B, T, HV, 1 or V]
    spans = seq_spans(B, T, cu_seqlens)
    o = np.zeros((B, T, HV, V), f)
    ht = np.zeros((len(spans), HV, K, V), f)
    pick = lambda x, b, t: None if x is None else x[b, t]   # noqa: E731
    for n, (b, bos, eos) in enumerate(spans):
        S = np.zeros((HV, K, V), f)
        if initial_state is not None:
            S = S + np.asarray(initial_state[n], f)
        for t in range(bos, eos):
            decay = _rec_decay(f, pick(g, b, t), pick(gk, b, t), pick(gv, b, t), HV, K, V)
            S, o[b, t] = _rec_token(S, decay, qf[b, t], kf[b, t], vf[b, t], bf[b, t])
        ht[n] = S
    return cast(o, o_dtype) if dtype != "fp64" else o, ht


def causal_conv1d(x, weight, bias=None, initial_state=None, cu_seqlens=None, activation=None,
                  l2norm_head_dim=0, dtype: str = "fp32"):
    """Short causal convolution per channel (fla modules/convolution.py:54-141, :410-458):
    y[t, d] = act(sum_i weight[d, i] x~[t - W + 1 + i, d] + bias[d]), x~ = x inside the
    sequence, else the cache initial_state [N, D, W] (slot W-1 the most recent input),
    else 0; fp32 arithmetic, y rounded to ``dtype`` (x's storage dtype).  With
    ``l2norm_head_dim`` the rounded y is L2-normalised per head (l2norm.py:115-118)
    and rounded again.  Returns (y [B, T, D], final_state [N, D, W]) where final_state
    is the last W entries of [cache, x] per sequence (convolution.py:539-574).
    """
    B, T, D = x.shape
    W = weight.shape[1]
    xf = np.asarray(x, np.float64)
    wf = np.asarray(weight, np.float64)
    spans = seq_spans(B, T, cu_seqlens)
    y = np.zeros((B, T, D), np.float64)
    final = np.zeros((len(spans), D, W), np.float64)
    for n, (b, bos, eos) in enumerate(spans):
        cache = np.zeros((W, D)) if initial_state is None else np.asarray(initial_state[n], np.float64).T
        ext = np.concatenate([cache, xf[b, bos:eos]], axis=0)          # [W + T_n, D], x~ from slot 0
        for t in range(eos - bos):
            win = ext[t + 1:t + 1 + W]                                  # x~[t - W + 1 .. t]
            y[b, bos + t] = np.sum(win * wf.T, axis=0)
        final[n] = ext[-W:].T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    y = y.astype(np.float32)                                            # fp32 accumulation
    if activation in ("silu", "swish"):
        y = y / (1.0 + np.exp(-y))
    y = cast(y, dtype)
    if l2norm_head_dim:
        yh = y.reshape(B, T, D // l2norm_head_dim, l2norm_head_dim)
        yh = yh / np.sqrt(np.sum(yh * yh, axis=-1, keepdims=True, dtype=np.float32) + np.float32(1e-6))
        y = cast(yh.reshape(B, T, D), dtype)
    return y, cast(final.astype(np.float32), dtype)


def gdn_gates(a, b, A_log, dt_bias, allow_neg_eigval=False, b_dtype: str = "fp32"):
    """Gates of the GatedDeltaNet layer (layers/gated_deltanet.py:265-271): g = -exp(A_log)
    softplus(a + dt_bias) in fp32 (torch softplus, threshold 20) and beta = sigmoid(b) rounded
    to b's dtype, doubled with allow_neg_eigval.  a, b: [..., HV]; returns (g, beta)."""
    z = np.asarray(a, np.float32) + np.asarray(dt_bias, np.float32)
    sp = np.where(z > 20, z, np.log1p(np.exp(np.minimum(z, 20)))).astype(np.float32)
    g = (-np.exp(np.asarray(A_log, np.float32)) * sp).astype(np.float32)
    beta = cast(1.0 / (1.0 + np.exp(-np.asarray(b, np.float64))), b_dtype)
    if allow_neg_eigval:
        beta = beta * 2
    return g, beta


def naive_recurrent(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None, dtype: str = "fp64"):
    """Token-by-token gated delta rule, per sequence (gated_delta_product/naive.py:23-35,
    fused_recurrent.py:88-119):

        S <- exp(g_t) S ;  v'_t = beta_t (v_t - S^T k_t) ;  S <- S + k_t v'_t^T ;  o_t = scale * S^T q_t
    Returns (o [B, T, H, V], ht [N, H, K, V]) in float64 (or float32 for dtype="fp32").
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    f = np.float64 if dtype == "fp64" else np.float32
    if scale is None:
        scale = K ** -0.5
    qf, kf, vf, gf, bf = (np.asarray(x, f) for x in (q, k, v, g, beta))
    spans = seq_spans(B, T, cu_seqlens)
    o = np.zeros((B, T, H, V), f)
    ht = np.zeros((len(spans), H, K, V), f)
    for n, (b, bos, eos) in enumerate(spans):
        S = np.zeros((H, K, V), f)
        if initial_state is not None:
            S = S + np.asarray(initial_state[n], f)
        for t in range(bos, eos):
            S = S * np.exp(gf[b, t])[:, None, None]
            kt = kf[b, t]                                           # [H, K]
            vp = bf[b, t][:, None] * (vf[b, t] - np.einsum("hkv,hk->hv", S, kt))
            S = S + kt[:, :, None] * vp[:, None, :]
            o[b, t] = scale * np.einsum("hkv,hk->hv", S, qf[b, t])
        ht[n] = S
    return o, ht
