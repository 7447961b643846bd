"""Host side of the token-by-token gated delta rule (the layer's short-sequence mode).

``fused_recurrent_gated_delta_rule`` keeps the signature, argument meaning,
defaults and error behaviour of the reference
(kairos/third_party/fla/ops/gated_delta_rule/fused_recurrent.py:238-349) and
runs through the HIP kernel behind ``kairos_gdn_fused_recurrent_fwd``.  The
GatedDeltaNet layer calls it instead of the chunked op when q_len <= 64
(fla/layers/gated_deltanet.py:220,287-297).  There is no other compute path.
"""
from __future__ import annotations

import torch

from . import _lib
from .chunk import _code, _prepare_cu_seqlens, _ptr, _require_device, _stream


def _opt_code(t, what):
    return _code(t, what) if t is not None else _lib.F32


def fused_recurrent_gated_delta_rule_fwd(q, k, v, g=None, gk=None, gv=None, beta=None, scale=None,
                                         initial_state=None, output_final_state=False,
                                         use_qk_l2norm_in_kernel=False, cu_seqlens=None):
    """One native call (fused_recurrent.py:138-185).  Returns (o in v's dtype, final_state fp32 or None)."""
    dev = _require_device(q, k, v, g, gk, gv, beta, initial_state)
    B, T, H, K = k.shape
    HV, V = v.shape[2], v.shape[3]
    if q.shape != k.shape or v.shape[:2] != (B, T):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if HV % H != 0:
        raise ValueError(f"the value heads ({HV}) must be a multiple of the q/k heads ({H})")
    if g is not None and tuple(g.shape) != (B, T, HV):
        raise ValueError(f"g must have shape {(B, T, HV)}, got {tuple(g.shape)}")
    if gk is not None and tuple(gk.shape) != (B, T, HV, K):
        raise ValueError(f"gk must have shape {(B, T, HV, K)}, got {tuple(gk.shape)}")
    if gv is not None and tuple(gv.shape) != (B, T, HV, V):
        raise ValueError(f"gv must have shape {(B, T, HV, V)}, got {tuple(gv.shape)}")
    headwise = 1
    if beta is not None:
        # the reference tells the two forms apart by rank (IS_BETA_HEADWISE = beta.ndim != v.ndim)
        headwise = int(beta.ndim != v.ndim)
        want = (B, T, HV) if headwise else (B, T, HV, V)
        if tuple(beta.shape) != want:
            raise ValueError(f"beta must have shape {want}, got {tuple(beta.shape)}")
    if k.dtype != q.dtype:
        raise TypeError("q and k must share a dtype")
    q, k, v = (x.contiguous() for x in (q, k, v))
    g, gk, gv, beta = (x.contiguous() if x is not None else None for x in (g, gk, gv, beta))
    n_seqs, cu = 0, None
    if cu_seqlens is not None:
        cu = _prepare_cu_seqlens(cu_seqlens, dev, T)
        n_seqs = cu.numel() - 1
    N = n_seqs if cu is not None else B
    h0, h0_dt = None, _lib.F32
    if initial_state is not None:
        if tuple(initial_state.shape) != (N, HV, K, V):
            raise ValueError(f"initial_state must have shape {(N, HV, K, V)}, got {tuple(initial_state.shape)}")
        h0 = initial_state if initial_state.dtype in (torch.float32, torch.bfloat16) else initial_state.float()
        h0 = h0.contiguous()
        h0_dt = _code(h0, "initial_state")
    o = torch.empty_like(v)
    ht = torch.empty(N, HV, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    if scale is None:
        scale = K ** -0.5
    _lib.call("kairos_gdn_fused_recurrent_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(gk), _ptr(gv), _ptr(beta),
              _ptr(h0), _ptr(o), _ptr(ht), _ptr(cu), n_seqs, B, T, H, HV, K, V, _code(q, "q"), _code(v, "v"),
              _opt_code(g, "g"), _opt_code(gk, "gk"), _opt_code(gv, "gv"), _opt_code(beta, "beta"), headwise, h0_dt,
              float(scale), int(bool(use_qk_l2norm_in_kernel)), _stream(dev))
    return o, ht


class FusedRecurrentFunction(torch.autograd.Function):
    """Forward-only, as the reference's (fused_recurrent.py:192-235, whose backward raises)."""

    @staticmethod
    def forward(ctx, q, k, v, g=None, gk=None, gv=None, beta=None, scale=None, initial_state=None,
                output_final_state=False, use_qk_l2norm_in_kernel=False, cu_seqlens=None):
        return fused_recurrent_gated_delta_rule_fwd(q, k, v, g, gk, gv, beta, scale, initial_state,
                                                    output_final_state, use_qk_l2norm_in_kernel, cu_seqlens)

    @staticmethod
    def backward(ctx, do, dht):
        raise NotImplementedError(
            "Backward pass is not implemented yet and we do not have plans to implement it "
            "because we haven't figured out how to compute dg without materializing the full "
            "hidden states for all time steps.",
        )


@torch.compiler.disable
def fused_recurrent_gated_delta_rule(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor | None = None,
                                     gk: torch.Tensor | None = None, gv: torch.Tensor | None = None,
                                     beta: torch.Tensor | None = None, scale: float = None,
                                     initial_state: torch.Tensor = None, output_final_state: bool = False,
                                     use_qk_l2norm_in_kernel: bool = False,
                                     cu_seqlens: torch.LongTensor | None = None):
    r"""Token-by-token gated delta rule on MI355X (contract of fused_recurrent.py:238-349).

    q, k [B, T, H, K]; v [B, T, HV, V] (HV a multiple of H); g [B, T, HV], gk
    [B, T, HV, K], gv [B, T, HV, V] log-space decays (each optional); beta
    [B, T, HV] or [B, T, HV, V] (default ones); initial_state [N, HV, K, V];
    cu_seqlens int64 [N+1] for packed variable-length input (B must be 1).
    Returns (o [B, T, HV, V] in v's dtype, final_state [N, HV, K, V] fp32 or None).
    """
    if cu_seqlens is not None:
        if q.shape[0] != 1:
            raise ValueError(
                f"The batch size is expected to be 1 rather than {q.shape[0]} when using `cu_seqlens`."
                f"Please flatten variable-length inputs before processing.",
            )
        if initial_state is not None and initial_state.shape[0] != len(cu_seqlens) - 1:
            raise ValueError(
                f"The number of initial states is expected to be equal to the number of input sequences, "
                f"i.e., {len(cu_seqlens) - 1} rather than {initial_state.shape[0]}.",
            )
    if scale is None:
        scale = k.shape[-1] ** -0.5
    # beta=None means ones (fused_recurrent.py:332-333); the kernel takes a null beta as ones
    return FusedRecurrentFunction.apply(q, k, v, g, gk, gv, beta, scale, initial_state, output_final_state,
                                        use_qk_l2norm_in_kernel, cu_seqlens)
