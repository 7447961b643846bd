"""Gated RMSNorm: the output epilogue of the GatedDeltaNet layer.

Mirrors ``rms_norm_gated`` and ``FusedRMSNormGated`` of the vendored fla
(kairos/third_party/fla/modules/fused_norm_gate.py:875-899, :1024-1088), the
layer's ``o_norm`` (fla/layers/gated_deltanet.py:197, :311).  The forward runs
in the HIP kernel behind ``kairos_gdn_rms_norm_gated`` (include/kairos_gdn.h);
there is no other compute path.

Built: the RMS path without residual (what the GatedDeltaNet layer uses),
activations 'swish' / 'silu' / 'sigmoid', optional weight and bias, fp32 or
bf16 x and gate, last dim a multiple of 8 up to 512.  The residual / prenorm
variants and the backward raise.
"""
from __future__ import annotations

import torch
from torch import nn

from . import _lib
from .chunk import _code, _ptr, _require_device, _stream

_ACT = {"swish": _lib.ACT_SWISH, "silu": _lib.ACT_SWISH, "sigmoid": _lib.ACT_SIGMOID}


def rms_norm_gated_fwd(x: torch.Tensor, g: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
                       activation: str = "swish", eps: float = 1e-6, return_rstd: bool = False):
    """layer_norm_gated_fwd with is_rms_norm=True and no residual
    (fused_norm_gate.py:449-525): returns y (x's dtype) and, if asked, rstd [rows] fp32."""
    if activation not in _ACT:
        raise ValueError(f"Unsupported activation: {activation}")
    if g.shape != x.shape:
        raise ValueError(f"gate shape {tuple(g.shape)} != input shape {tuple(x.shape)}")
    D = x.shape[-1]
    for name, p in (("weight", weight), ("bias", bias)):
        if p is not None and tuple(p.shape) != (D,):
            raise ValueError(f"{name} must have shape ({D},), got {tuple(p.shape)}")
    if weight is not None and bias is not None and weight.dtype != bias.dtype:
        raise TypeError("weight and bias must share a dtype")
    _require_device(x, g, weight, bias)
    x = x.contiguous()
    g = g.contiguous()
    weight = weight.contiguous() if weight is not None else None
    bias = bias.contiguous() if bias is not None else None
    rows = x.numel() // D if D else 0
    y = torch.empty_like(x)
    rstd = torch.empty(rows, dtype=torch.float32, device=x.device) if return_rstd else None
    pw = weight if weight is not None else bias
    w_code = _code(pw, "weight") if pw is not None else _lib.F32
    _lib.call("kairos_gdn_rms_norm_gated", _ptr(x), _ptr(g), _ptr(weight), _ptr(bias), _ptr(y), _ptr(rstd),
              _code(x, "x"), _code(g, "g"), w_code, rows, D, float(eps), _ACT[activation], _stream(x.device))
    return (y, rstd) if return_rstd else y


class _RMSNormGatedFunction(torch.autograd.Function):
    """Forward of LayerNormGatedFunction (fused_norm_gate.py:647-703) on the RMS path."""

    @staticmethod
    def forward(ctx, x, g, weight, bias, activation, eps):
        shape = x.shape
        y = rms_norm_gated_fwd(x.reshape(-1, shape[-1]), g.reshape(-1, g.shape[-1]), weight, bias, activation, eps)
        return y.reshape(shape)

    @staticmethod
    def backward(ctx, dy):
        raise NotImplementedError("kairos_gdn builds the gated RMSNorm forward only (inference)")


def rms_norm_gated(x: torch.Tensor, g: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
                   activation: str = "swish", residual: torch.Tensor | None = None, prenorm: bool = False,
                   residual_in_fp32: bool = False, eps: float = 1e-6, tp_group=None) -> torch.Tensor:
    """fla modules/fused_norm_gate.py:875-899 (same arguments and defaults)."""
    if residual is not None or prenorm:
        raise NotImplementedError("kairos_gdn builds rms_norm_gated without residual / prenorm")
    if tp_group is not None:
        raise NotImplementedError("kairos_gdn runs on one GPU: tp_group is not supported")
    return _RMSNormGatedFunction.apply(x, g, weight, bias, activation, eps)


class FusedRMSNormGated(nn.Module):
    """fla modules/fused_norm_gate.py:1024-1088: y = RMSNorm(x) * weight * act(g)."""

    def __init__(self, hidden_size: int, elementwise_affine: bool = True, eps: float = 1e-5,
                 activation: str = "swish", device: torch.device | None = None, dtype: torch.dtype | None = None):
        factory_kwargs = {"device": device, "dtype": dtype}
        super().__init__()
        self.hidden_size = hidden_size
        self.elementwise_affine = elementwise_affine
        self.eps = eps
        self.activation = activation
        if self.activation not in ["swish", "silu", "sigmoid"]:
            raise ValueError(f"Unsupported activation: {self.activation}")
        if elementwise_affine:
            self.weight = nn.Parameter(torch.empty(hidden_size, **factory_kwargs))
        else:
            self.register_parameter("weight", None)
        self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self):
        if self.elementwise_affine:
            nn.init.ones_(self.weight)

    def extra_repr(self) -> str:
        parts = [str(self.hidden_size), f"eps={self.eps}", f"activation={self.activation}"]
        if not self.elementwise_affine:
            parts.insert(1, "elementwise_affine=False")
        return ", ".join(parts)

    def forward(self, x: torch.Tensor, g: torch.Tensor, residual: torch.Tensor | None = None, prenorm: bool = False,
                residual_in_fp32: bool = False, tp_group=None) -> torch.Tensor:
        return rms_norm_gated(x, g, self.weight, self.bias, self.activation, residual=residual, eps=self.eps,
                              prenorm=prenorm, residual_in_fp32=residual_in_fp32, tp_group=tp_group)
