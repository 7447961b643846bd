"""fp32 torch-CPU restatement of the chunked GatedDeltaNet forward -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` and ``bench.py``'s CPU-baseline leg may import this module; the
product path never calls it.  It is the CPU path timed beside the GPU: the
reference algorithm of flash-linear-attention 0.4.0 (vendored in
``kairos/third_party/fla``) written with torch-CPU batched matmuls, all in the
floating type of its inputs (float32 for the baseline, float64 in the tests
that pin it), without the bf16 cast points of ``gdn_oracle``:

  stage                      reference
  -------------------------  ------------------------------------------------
  chunk_local_cumsum         ops/utils/cumsum.py:27-65
  chunk_scaled_dot_kkt       ops/common/chunk_scaled_dot_kkt.py:57-73
  solve_tril                 ops/utils/solve_tril.py:184-331 ((I + A)^-1, here by
                             torch.linalg.solve_triangular)
  recompute_w_u              ops/gated_delta_rule/wy_fast.py:55-81
  chunk_fwd_h                ops/common/chunk_delta_h.py:113-224 (serial over chunks,
                             batched over heads)
  chunk_fwd_o                ops/common/chunk_o.py:84-128
  orchestration              ops/gated_delta_rule/chunk.py:16-67

Pinned by tests/test_oracle.py: in float64 it equals the fp64 token
recurrence ``gdn_oracle.naive_recurrent`` (< 1e-10, ragged tails, varlen, h0),
and in float32 it matches ``gdn_oracle.chunk_gated_delta_rule(dtype="fp32")``.
"""
from __future__ import annotations

import torch

CHUNK = 64


def _one_sequence(q, k, v, g, beta, scale, h0, chunk):
    """q, k [T, H, K]; v [T, H, V]; g, beta [T, H]; h0 [H, K, V] or None -> (o [T, H, V], ht [H, K, V])."""
    T, H, K = q.shape
    V = v.shape[-1]
    dt = q.dtype
    nc = (T + chunk - 1) // chunk
    pad = nc * chunk - T

    def chunked(x):                          # [T, H, ...] -> [H, NC, C, ...], zero rows past T
        if pad:
            x = torch.cat([x, x.new_zeros((pad,) + tuple(x.shape[1:]))], 0)
        x = x.reshape(nc, chunk, *x.shape[1:])
        return x.movedim(2, 0).contiguous()

    qc, kc, vc = chunked(q), chunked(k), chunked(v)
    gc = chunked(g).cumsum(-1)               # chunk-local cumsum; padded rows repeat the last value
    bc = chunked(beta)
    # A = beta_i exp(gc_i - gc_j) k_i.k_j, strictly lower (padded rows are zero through beta = 0)
    strict = torch.ones(chunk, chunk, dtype=torch.bool).tril(-1)
    A = (kc @ kc.transpose(-1, -2)) * torch.exp(gc[..., :, None] - gc[..., None, :]) * bc[..., :, None]
    A = torch.where(strict, A, A.new_zeros(()))
    eye = torch.eye(chunk, dtype=dt)
    Ai = torch.linalg.solve_triangular(eye + A, eye.expand_as(A), upper=False, unitriangular=True)
    w = Ai @ (kc * (bc * torch.exp(gc))[..., None])
    u = Ai @ (vc * bc[..., None])
    # Aqk = q_i.k_j exp(gc_i - gc_j), lower with the diagonal
    lower = torch.ones(chunk, chunk, dtype=torch.bool).tril()
    Aqk = torch.where(lower, (qc @ kc.transpose(-1, -2)) * torch.exp(gc[..., :, None] - gc[..., None, :]),
                      A.new_zeros(()))
    valid = torch.arange(nc * chunk).reshape(nc, chunk) < T          # [NC, C]
    S = h0.to(dt).clone() if h0 is not None else torch.zeros(H, K, V, dtype=dt)
    o = torch.empty(H, nc, chunk, V, dtype=dt)
    for c in range(nc):
        gcc = gc[:, c]                                                # [H, C]
        gl = gcc[:, -1]                                               # [H] (padding repeats the last valid gc)
        vp = u[:, c] - w[:, c] @ S                                    # [H, C, V]
        o[:, c] = (qc[:, c] @ S) * torch.exp(gcc)[..., None] + Aqk[:, c] @ vp
        gate = torch.where(valid[c], torch.exp(gl[:, None] - gcc), gcc.new_zeros(()))
        S = S * torch.exp(gl)[:, None, None] + kc[:, c].transpose(-1, -2) @ (vp * gate[..., None])
    o = (o * scale).reshape(H, nc * chunk, V)[:, :T].movedim(0, 1)
    return o, S


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None, cu_seqlens=None, chunk: int = CHUNK):
    """Chunked forward on CPU tensors of one floating type (chunk.py:16-67).

    q, k [B, T, H, K]; v [B, T, H, V]; g, beta [B, T, H]; initial_state [N, H, K, V]
    or None; cu_seqlens (ints, B == 1) or None.  Returns (o [B, T, H, V], final_state
    [N, H, K, V]) in the inputs' type.
    """
    B, T, H, K = q.shape
    if scale is None:
        scale = K ** -0.5
    if cu_seqlens is None:
        spans = [(b, 0, T) for b in range(B)]
    else:
        cu = [int(x) for x in cu_seqlens]
        spans = [(0, cu[i], cu[i + 1]) for i in range(len(cu) - 1)]
    o = torch.zeros(B, T, H, v.shape[-1], dtype=q.dtype)
    ht = torch.zeros(len(spans), H, K, v.shape[-1], dtype=q.dtype)
    for n, (b, bos, eos) in enumerate(spans):
        h0 = initial_state[n] if initial_state is not None else None
        if eos == bos:
            ht[n] = h0 if h0 is not None else 0
            continue
        o[b, bos:eos], ht[n] = _one_sequence(q[b, bos:eos], k[b, bos:eos], v[b, bos:eos], g[b, bos:eos],
                                             beta[b, bos:eos], scale, h0, chunk)
    return o, ht
