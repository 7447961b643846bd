"""Host side of the GatedDeltaNet layer's prologue: short causal convolution and gates.

``causal_conv1d`` and ``ShortConvolution`` keep the signature, argument meaning
and cache behaviour of the reference (kairos/third_party/fla/modules/convolution.py:
692-790 and :801-1100, Triton backend) and run through the HIP kernels behind
``kairos_gdn_causal_conv1d_fwd``; ``gdn_gates`` computes the layer's decay and
write-strength gates (fla/layers/gated_deltanet.py:265-271) through
``kairos_gdn_gates_fwd``.  The layer builds ShortConvolution in its constructor
(gated_deltanet.py:176-189), so ``swap.install()`` rebinds that class name.
There is no other compute path.
"""
from __future__ import annotations

import warnings

import torch
import torch.nn as nn

from . import _lib
from .chunk import _code, _prepare_cu_seqlens, _ptr, _require_device, _stream


def causal_conv1d(x: torch.Tensor, weight: torch.Tensor | None = None, bias: torch.Tensor | None = None,
                  residual: torch.Tensor | None = None, initial_state: torch.Tensor | None = None,
                  output_final_state: bool | None = False, activation: str | None = None,
                  backend: str | None = 'triton', cu_seqlens: torch.Tensor | None = None,
                  l2norm_head_dim: int = 0, **kwargs):
    """Causal depthwise convolution over time (contract of convolution.py:692-790).

    x [B, T, D]; weight [D, W] (W <= 4); bias [D]; initial_state [N, D, W] (the cache
    of the previous call); cu_seqlens int64 [N+1] for packed sequences (B must be 1).
    Returns (y [B, T, D] in x's dtype, final_state [N, D, W] or None).
    ``l2norm_head_dim`` (extension): L2-normalise y per head of that many channels,
    the normalisation the layer otherwise asks the chunked op for.
    """
    if weight is None:
        raise NotImplementedError("causal_conv1d without a weight is not built (the layer always has one)")
    if residual is not None:
        raise NotImplementedError("causal_conv1d with a residual is not built (the GatedDeltaNet layer passes none)")
    if activation not in (None, 'silu', 'swish'):
        raise ValueError(f"Activation `{activation}` not supported yet.")
    dev = _require_device(x, weight, bias, initial_state)
    shape = x.shape
    if x.shape[-1] != weight.shape[0]:
        x = x.reshape(x.shape[0], x.shape[1], -1)
    B, T, D = x.shape
    W = weight.shape[1]
    if cu_seqlens is not None and B != 1:
        raise ValueError(f"The batch size is expected to be 1 rather than {B} when using `cu_seqlens`.")
    x = x.contiguous()
    weight = weight.contiguous()
    if weight.data_ptr() % 16:                       # the kernel reads the taps 16 bytes at a time
        weight = weight.clone()
    bias = bias.contiguous() if bias is not None else None
    if bias is not None and bias.dtype != weight.dtype:
        bias = bias.to(weight.dtype)
    n_seqs, cu = 0, None
    if cu_seqlens is not None:
        cu = _prepare_cu_seqlens(cu_seqlens, dev, T)
        n_seqs = cu.numel() - 1
    N = n_seqs if cu is not None else B
    h0 = None
    if initial_state is not None:
        if tuple(initial_state.shape) != (N, D, W):
            raise ValueError(f"initial_state must have shape {(N, D, W)}, got {tuple(initial_state.shape)}")
        h0 = initial_state.to(x.dtype).contiguous()
    y = torch.empty_like(x)
    ht = torch.empty(N, D, W, device=dev, dtype=x.dtype) if output_final_state else None
    _lib.call("kairos_gdn_causal_conv1d_fwd", _ptr(x), _ptr(weight), _ptr(bias), _ptr(h0), _ptr(y), _ptr(ht),
              _ptr(cu), n_seqs, B, T, D, W, _code(x, "x"), _code(weight, "weight"),
              int(activation in ('silu', 'swish')), int(l2norm_head_dim), _stream(dev))
    return y.view(shape), ht


class ShortConvolution(nn.Conv1d):
    """Depthwise causal convolution layer (the reference's ShortConvolution, convolution.py:801-1100).

    Same parameters (weight [D, 1, W], optional bias) and forward contract:
    forward(x, residual=None, mask=None, cache=None, output_final_state=False,
    cu_seqlens=None) -> (y, cache).  In the decoding case (one token per
    sequence) the cache is updated in place, as the reference's step().
    Tensor-parallel splitting of the reference's constructor is not built.
    """

    def __init__(self, hidden_size: int, kernel_size: int, bias: bool = False, activation: str | None = 'silu',
                 backend: str | None = 'triton', device=None, dtype=None, tp_num_splits: int = 1,
                 tp_chunk_list: list | None = None, tp_group=None, **kwargs):
        super().__init__(in_channels=hidden_size, out_channels=hidden_size, kernel_size=kernel_size,
                         groups=hidden_size, bias=bias, padding=kernel_size - 1, device=device, dtype=dtype)
        if tp_num_splits > 1 or tp_chunk_list is not None:
            raise NotImplementedError("tensor-parallel ShortConvolution is not built")
        self.hidden_size = hidden_size
        self.activation = None
        if activation is not None:
            assert activation in ['silu', 'swish'], f"Activation `{activation}` not supported yet."
            self.activation = activation
        if 'use_fast_conv1d' in kwargs:
            warnings.warn(
                "The `use_fast_conv1d` parameter is deprecated and will be ignored. "
                "Please use the `backend` parameter instead.",
            )
        if backend not in ['cuda', 'triton']:
            raise ValueError(f"Invalid backend: {backend}, must be one of ['cuda', 'triton']")
        self.backend = backend

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None, mask: torch.Tensor | None = None,
                cache: torch.Tensor | None = None, output_final_state: bool = False,
                cu_seqlens: torch.LongTensor | None = None, **kwargs):
        B, T, *_ = x.shape
        N = B if cu_seqlens is None else len(cu_seqlens) - 1
        if mask is not None:
            if cu_seqlens is not None:
                raise ValueError("`mask` and `cu_seqlens` cannot be provided at the same time")
            x = x.mul_(mask.unsqueeze(-1))
        weight = self.weight.reshape(self.hidden_size, -1)
        if B * T == N:                                   # decoding: the cache is updated in place
            if output_final_state and cache is None:
                cache = x.new_zeros(N, self.hidden_size, weight.shape[1])
            y, new_cache = causal_conv1d(x, weight, self.bias, residual, cache, cache is not None, self.activation,
                                         cu_seqlens=cu_seqlens)
            if cache is not None:
                cache.copy_(new_cache)
            return y, cache
        return causal_conv1d(x, weight, self.bias, residual, cache, output_final_state, self.activation,
                             cu_seqlens=cu_seqlens)

    @property
    def state_size(self) -> int:
        return self.hidden_size * self.kernel_size[0]


def gdn_gates(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor,
              allow_neg_eigval: bool = False):
    """g = -exp(A_log) * softplus(a + dt_bias) (fp32) and beta = sigmoid(b) (b's dtype, x2 with
    allow_neg_eigval): the gate lines of GatedDeltaNet.forward (gated_deltanet.py:265-271), with
    a = a_proj(h), b = b_proj(h) of shape [..., HV] and the layer's A_log, dt_bias [HV]."""
    dev = _require_device(a, b, A_log, dt_bias)
    if a.shape != b.shape:
        raise ValueError(f"a {tuple(a.shape)} and b {tuple(b.shape)} must have one shape")
    HV = a.shape[-1]
    if A_log.numel() != HV or dt_bias.numel() != HV:
        raise ValueError(f"A_log and dt_bias must have {HV} entries")
    pdt = torch.float32 if torch.float32 in (A_log.dtype, dt_bias.dtype) else A_log.dtype
    A_log = A_log.to(pdt).contiguous()
    dt_bias = dt_bias.to(pdt).contiguous()
    a, b = a.contiguous(), b.contiguous()
    g = torch.empty(a.shape, device=dev, dtype=torch.float32)
    beta = torch.empty_like(b)
    _lib.call("kairos_gdn_gates_fwd", _ptr(a), _ptr(b), _ptr(A_log), _ptr(dt_bias), _ptr(g), _ptr(beta),
              a.numel() // HV, HV, _code(a, "a"), _code(b, "b"), _code(A_log, "A_log"), int(bool(allow_neg_eigval)),
              _stream(dev))
    return g, beta
