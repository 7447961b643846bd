"""Host side of the MI355X chunked GatedDeltaNet forward.

``chunk_gated_delta_rule`` keeps the signature, argument meaning, defaults and
error behaviour of the reference entry point
(kairos/third_party/fla/ops/gated_delta_rule/chunk.py:217-323) and runs the
forward through the HIP kernels of libkairos_gdn.so.  PyTorch only provides
device memory and the current stream.  There is no other compute path: on a
machine without the library or a HIP device every call raises.

The stage functions below (``chunk_local_cumsum``, ``prepare_wy``, ``fwd_h``,
``fwd_o``, ``l2norm_fwd``) expose the individual kernels with the reference's
stage semantics, for parity tests and for callers that compose stages.
"""
from __future__ import annotations

import warnings

import torch

from . import _lib

CHUNK = 64

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
_FP8 = getattr(torch, "float8_e4m3fn", None)
if _FP8 is not None:
    _DTYPES[_FP8] = _lib.F8E4M3


def _code(t: torch.Tensor, what: str) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype} (fp32, bf16, or fp8 e4m3 for q/k)") from None


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_device(*tensors):
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "kairos_gdn runs on a HIP device only (tensor on %s); there is no CPU path" % t.device)
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"all tensors must be on one device ({dev} vs {t.device})")
    return dev


_validated_cu: tuple | None = None


def _prepare_cu_seqlens(cu_seqlens: torch.Tensor, device: torch.device, T: int) -> torch.Tensor:
    """int64 device copy of cu_seqlens, checked once per tensor object and version.

    The reference reads cu_seqlens on the host as well (prepare_chunk_indices
    calls .tolist(), fla/ops/utils/index.py:118, cached by identity in
    fla/utils.py:96-133); the same check here guards the kernels against
    offsets outside [0, T].  The cache key includes the tensor's version
    counter, so an in-place edit of a reused buffer is checked again.  A tensor
    made under ``torch.inference_mode()`` has no version counter: it is checked
    on every call.
    """
    global _validated_cu
    cu = cu_seqlens
    if cu.dim() != 1 or cu.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D tensor with at least two entries")
    version = None
    if not cu_seqlens.is_inference():
        try:
            version = cu_seqlens._version
        except RuntimeError:                      # no version counter to key on
            version = None
    key = (cu_seqlens, version, T)
    if (version is None or _validated_cu is None or _validated_cu[0] is not key[0] or _validated_cu[1] != key[1]
            or _validated_cu[2] != key[2]):
        vals = cu.detach().to("cpu", torch.int64)
        if int(vals[0]) != 0 or int(vals[-1]) != T or bool((vals[1:] < vals[:-1]).any()):
            raise ValueError(
                f"cu_seqlens must start at 0, end at T={T} and be non-decreasing (got {vals.tolist()[:8]}...)")
        _validated_cu = key if version is not None else None
    return cu.to(device=device, dtype=torch.int64).contiguous()


def _f16_as_f32(*xs):
    """fp16 tensors as fp32 (others unchanged); with fp16 q, k or v all three are taken in fp32.

    The reference op is dtype-generic (chunk.py:149-186 under autocast_custom_fwd): with fp16
    inputs its kernels take fp16 operands and round Ai, w, u, h, v_new and o to fp16.  The
    kernels here are built for bf16 and fp32 storage, so fp16 inputs run the fp32 kernels on
    exact fp32 copies and o is rounded to fp16 once, at the end: no fp16 intermediate rounding,
    hence at least as close to the exact recurrence as the reference's fp16 path.
    """
    return tuple(x.float() if (x is not None and x.dtype == torch.float16) else x for x in xs)


def _scales(q_scale, k_scale, H, device, fp8: bool):
    if not fp8:
        return None, None
    if q_scale is None or k_scale is None:
        raise ValueError("fp8 q/k need per-head q_scale and k_scale of shape [H]")
    qs = q_scale.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    ks = k_scale.to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    if qs.numel() != H or ks.numel() != H:
        raise ValueError(f"q_scale / k_scale must have H={H} entries")
    return qs, ks


def chunk_gated_delta_rule_fwd(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens=None,
                               use_qk_l2norm_in_kernel=False, q_scale=None, k_scale=None, _norm=None):
    """One native call: [q/k L2 norm] -> prepare -> state recurrence -> output.

    Mirrors chunk_gated_delta_rule_fwd (chunk.py:16-67) plus the optional
    in-kernel L2 norm of ChunkGatedDeltaRuleFunction.forward (chunk.py:168-170),
    with the same positional arguments.  Returns (o in v's dtype, final_state
    fp32 or None); the reference returns (g, o, A, final_state), the cumsummed
    gates and A being its saved intermediates, which this library recomputes
    in the backward instead of keeping.  ``_norm`` (gate,
    weight, bias, eps, activation code) turns o into the layer's gated RMSNorm
    of o (chunk_gated_delta_rule_gated_norm).
    """
    dev = _require_device(q, k, v, g, beta, initial_state)
    B, T, H, K = q.shape
    V = v.shape[-1]
    if torch.float16 in (q.dtype, k.dtype, v.dtype):
        if _norm is not None:
            raise TypeError("the fused gated norm takes bf16 or fp32 q/k/v (fp16 given)")
        if q.dtype != k.dtype:
            raise TypeError("q and k must share a dtype")
        out_dt = v.dtype
        o, ht = chunk_gated_delta_rule_fwd(q.float(), k.float(), v.float(), *_f16_as_f32(g, beta), scale,
                                           *_f16_as_f32(initial_state), output_final_state, cu_seqlens,
                                           use_qk_l2norm_in_kernel, q_scale, k_scale)
        return o.to(out_dt), ht
    if k.shape != q.shape or v.shape[:3] != (B, T, H) or g.shape != (B, T, H) or beta.shape != (B, T, H):
        raise ValueError(
            f"shape mismatch: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}, g {tuple(g.shape)}, "
            f"beta {tuple(beta.shape)}")
    if k.dtype != q.dtype:
        raise TypeError("q and k must share a dtype")
    qk_dt, v_dt = _code(q, "q"), _code(v, "v")
    g_dt, b_dt = _code(g, "g"), _code(beta, "beta")
    fp8 = qk_dt == _lib.F8E4M3
    qs, ks = _scales(q_scale, k_scale, H, dev, fp8)
    q, k, v, g, beta = (x.contiguous() for x in (q, k, v, g, beta))
    n_seqs, cu = 0, None
    if cu_seqlens is not None:
        cu = _prepare_cu_seqlens(cu_seqlens, dev, T)
        n_seqs = cu.numel() - 1
    N = n_seqs if cu is not None else B
    h0, h0_dt = None, _lib.F32
    if initial_state is not None:
        if tuple(initial_state.shape) != (N, H, K, V):
            raise ValueError(f"initial_state must have shape {(N, H, K, V)}, got {tuple(initial_state.shape)}")
        h0 = initial_state
        if h0.dtype not in (torch.float32, torch.bfloat16):
            h0 = h0.float()
        h0 = h0.contiguous()
        h0_dt = _code(h0, "initial_state")
    o = torch.empty_like(v)
    ht = torch.empty(N, H, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    lib = _lib.load()
    ws_fn = lib.kairos_gdn_chunk_fwd_gated_norm_workspace_size if _norm is not None \
        else lib.kairos_gdn_chunk_fwd_workspace_size
    ws_bytes = ws_fn(B, T, H, K, V, n_seqs, qk_dt, v_dt, int(bool(use_qk_l2norm_in_kernel)))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    if _norm is not None:
        gate, nw, nb, eps, act = _norm
        w_dt = _code(nw if nw is not None else nb, "norm weight") if (nw is not None or nb is not None) else _lib.F32
        _lib.call("kairos_gdn_chunk_fwd_gated_norm", _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(qs),
                  _ptr(ks), _ptr(h0), _ptr(gate), _ptr(nw), _ptr(nb), _ptr(o), _ptr(ht), _ptr(cu), n_seqs, B, T, H,
                  K, V, qk_dt, v_dt, g_dt, b_dt, h0_dt, _code(gate, "gate"), w_dt, float(scale),
                  int(bool(use_qk_l2norm_in_kernel)), float(eps), act, _ptr(ws), ws_bytes, _stream(dev))
        return o, ht
    _lib.call("kairos_gdn_chunk_fwd", _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(qs), _ptr(ks),
              _ptr(h0), _ptr(o), _ptr(ht), _ptr(cu), n_seqs, B, T, H, K, V, qk_dt, v_dt, g_dt, b_dt, h0_dt,
              float(scale), int(bool(use_qk_l2norm_in_kernel)), _ptr(ws), ws_bytes, _stream(dev))
    return o, ht


_NORM_ACT = {"swish": _lib.ACT_SWISH, "silu": _lib.ACT_SWISH, "sigmoid": _lib.ACT_SIGMOID}


@torch.no_grad()
def chunk_gated_delta_rule_gated_norm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                                      beta: torch.Tensor, gate: torch.Tensor, norm_weight: torch.Tensor | None = None,
                                      norm_bias: torch.Tensor | None = None, scale: float | None = None,
                                      initial_state: torch.Tensor | None = None, output_final_state: bool = False,
                                      cu_seqlens: torch.Tensor | None = None, use_qk_l2norm_in_kernel: bool = False,
                                      activation: str = "swish", eps: float = 1e-5, q_scale=None, k_scale=None):
    """Forward of the GatedDeltaNet layer's recurrence and output norm in one call:
    ``o_norm(chunk_gated_delta_rule(q, k, v, g, beta, ...)[0], gate)``
    (fla layers/gated_deltanet.py:275-311, o_norm = FusedRMSNormGated on the
    RMS path without residual, modules/fused_norm_gate.py:42-127).

    Returns (y in v's dtype, final_state fp32 or None).  y equals
    ``rms_norm_gated(o, gate, norm_weight, norm_bias, activation, eps)`` of the
    plain forward's o (the norm reads o rounded to its dtype).  Forward only:
    training keeps the two calls, since the norm's backward needs o.  Where the
    segment scan runs (bf16, head dims 64 / 128) with a bf16 gate the norm is
    computed in the output kernel and o is never written.
    """
    if activation not in _NORM_ACT:
        raise ValueError(f"Unsupported activation: {activation}")
    V = v.shape[-1]
    if tuple(gate.shape) != tuple(v.shape):
        raise ValueError(f"gate shape {tuple(gate.shape)} != v shape {tuple(v.shape)}")
    for name, p in (("norm_weight", norm_weight), ("norm_bias", norm_bias)):
        if p is not None and tuple(p.shape) != (V,):
            raise ValueError(f"{name} must have shape ({V},), got {tuple(p.shape)}")
    if norm_weight is not None and norm_bias is not None and norm_weight.dtype != norm_bias.dtype:
        raise TypeError("norm_weight and norm_bias must share a dtype")
    _require_device(gate, norm_weight, norm_bias)
    if scale is None:
        scale = k.shape[-1] ** -0.5
    if cu_seqlens is not None and q.shape[0] != 1:
        raise ValueError(
            f"The batch size is expected to be 1 rather than {q.shape[0]} when using `cu_seqlens`."
            f"Please flatten variable-length inputs before processing.")
    gate = gate.contiguous()
    norm_weight = norm_weight.contiguous() if norm_weight is not None else None
    norm_bias = norm_bias.contiguous() if norm_bias is not None else None
    return chunk_gated_delta_rule_fwd(q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens,
                                      use_qk_l2norm_in_kernel, q_scale, k_scale,
                                      _norm=(gate, norm_weight, norm_bias, eps, _NORM_ACT[activation]))


@torch.no_grad()
def chunk_gated_delta_rule_conv(xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor, g: torch.Tensor,
                                beta: torch.Tensor, q_conv_weight: torch.Tensor, k_conv_weight: torch.Tensor,
                                v_conv_weight: torch.Tensor, q_conv_bias: torch.Tensor | None = None,
                                k_conv_bias: torch.Tensor | None = None, v_conv_bias: torch.Tensor | None = None,
                                scale: float | None = None, initial_state: torch.Tensor | None = None,
                                output_final_state: bool = False, conv_state: tuple | None = None,
                                output_conv_state: bool = False, cu_seqlens: torch.Tensor | None = None,
                                use_qk_l2norm_in_kernel: bool = False):
    """The GatedDeltaNet layer's prologue and recurrence in one call: the three ShortConvolutions
    (kernel size 4, SiLU; fla layers/gated_deltanet.py:234-253) on the projections and
    chunk_gated_delta_rule on their outputs (:275-285).

    xq, xk [B, T, H*K] and xv [B, T, H*V] are q_proj(h), k_proj(h), v_proj(h) in bf16; g, beta
    [B, T, H] as for chunk_gated_delta_rule; the conv weights are the ShortConvolutions' ([D, 1, 4]
    or [D, 4]) with optional biases; conv_state = (q, k, v) caches [N, D, 4] of the previous call or
    None.  Returns (o [B, T, H, V], final_state fp32 or None, (q, k, v) caches or None), the same
    values as causal_conv1d on each projection followed by chunk_gated_delta_rule.  At the layer's
    head dims (K = 256, V a multiple of 64) the convolution runs where the forward stages its rows
    (no convolved q / k / v round trip through HBM but q once); forward only.
    """
    dev = _require_device(xq, xk, xv, g, beta, q_conv_weight, k_conv_weight, v_conv_weight, initial_state)
    B, T, H = g.shape
    if beta.shape != g.shape:
        raise ValueError(f"beta {tuple(beta.shape)} and g {tuple(g.shape)} must have one shape")
    for n, x in (("xq", xq), ("xk", xk), ("xv", xv)):
        if x.dim() != 3 or x.shape[:2] != (B, T) or x.shape[-1] % H:
            raise ValueError(f"{n} must be [B, T, H * d] with B, T, H of g; got {tuple(x.shape)}")
        if x.dtype != torch.bfloat16:
            raise TypeError(f"{n}: the projections are taken in bf16 (got {x.dtype})")
    if xk.shape != xq.shape:
        raise ValueError(f"xq {tuple(xq.shape)} and xk {tuple(xk.shape)} must have one shape")
    K, V = xq.shape[-1] // H, xv.shape[-1] // H
    if cu_seqlens is not None and B != 1:
        raise ValueError(
            f"The batch size is expected to be 1 rather than {B} when using `cu_seqlens`."
            f"Please flatten variable-length inputs before processing.")
    if scale is None:
        scale = K ** -0.5
    ws3 = []
    for n, w, D in (("q", q_conv_weight, H * K), ("k", k_conv_weight, H * K), ("v", v_conv_weight, H * V)):
        w = w.reshape(w.shape[0], -1)
        if tuple(w.shape) != (D, 4):
            raise ValueError(f"{n}_conv_weight must hold [{D}, 4] taps (kernel size 4), got {tuple(w.shape)}")
        ws3.append(w.contiguous())
    w_dt = _code(ws3[0], "conv weight")
    if any(w.dtype != ws3[0].dtype for w in ws3):
        raise TypeError("the three conv weights must share a dtype")
    bs3 = []
    for n, b, D in (("q", q_conv_bias, H * K), ("k", k_conv_bias, H * K), ("v", v_conv_bias, H * V)):
        if b is not None:
            if b.numel() != D:
                raise ValueError(f"{n}_conv_bias must have {D} entries")
            b = b.reshape(-1).to(ws3[0].dtype).contiguous()
        bs3.append(b)
    n_seqs, cu = 0, None
    if cu_seqlens is not None:
        cu = _prepare_cu_seqlens(cu_seqlens, dev, T)
        n_seqs = cu.numel() - 1
    N = n_seqs if cu is not None else B
    cin = [None, None, None]
    if conv_state is not None:
        for i, (c, D) in enumerate(zip(conv_state, (H * K, H * K, H * V))):
            if c is not None:
                if tuple(c.shape) != (N, D, 4):
                    raise ValueError(f"conv_state[{i}] must have shape {(N, D, 4)}, got {tuple(c.shape)}")
                cin[i] = c.to(torch.bfloat16).contiguous()
    cout = [torch.empty(N, D, 4, device=dev, dtype=torch.bfloat16) for D in (H * K, H * K, H * V)] \
        if output_conv_state else [None, None, None]
    h0, h0_dt = None, _lib.F32
    if initial_state is not None:
        if tuple(initial_state.shape) != (N, H, K, V):
            raise ValueError(f"initial_state must have shape {(N, H, K, V)}, got {tuple(initial_state.shape)}")
        h0 = initial_state if initial_state.dtype in (torch.float32, torch.bfloat16) else initial_state.float()
        h0 = h0.contiguous()
        h0_dt = _code(h0, "initial_state")
    xq, xk, xv, g, beta = (x.contiguous() for x in (xq, xk, xv, g, beta))
    o = torch.empty(B, T, H, V, device=dev, dtype=torch.bfloat16)
    ht = torch.empty(N, H, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    l2 = int(bool(use_qk_l2norm_in_kernel))
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_fwd_conv_workspace_size(B, T, H, K, V, n_seqs, l2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _lib.call("kairos_gdn_chunk_fwd_conv", _ptr(xq), _ptr(xk), _ptr(xv), *(_ptr(w) for w in ws3),
              *(_ptr(b) for b in bs3), *(_ptr(c) for c in cin), *(_ptr(c) for c in cout), w_dt, _ptr(g),
              _ptr(beta), _ptr(h0), _ptr(o), _ptr(ht), _ptr(cu), n_seqs, B, T, H, K, V, _code(g, "g"),
              _code(beta, "beta"), h0_dt, float(scale), l2, _ptr(ws), ws_bytes, _stream(dev))
    return o, ht, (tuple(cout) if output_conv_state else None)


def chunk_gated_delta_rule_bwd_native(q, k, v, g, beta, scale, initial_state, do, dht, cu_seqlens=None,
                                      use_qk_l2norm_in_kernel=False):
    """One native call: gradients of chunk_gated_delta_rule (chunk.py:70-146, 188-213).

    Not the reference's ``chunk_gated_delta_rule_bwd(q, k, v, g, beta, A, ...)``,
    which takes the cumsummed gates and the forward's A: here ``g`` is the raw
    log-space gate and q, k are the forward's own inputs (before the optional
    in-op L2 norm); the library recomputes the norm, gc, Ai, w, u, h and v_new.
    Returns (dq, dk, dv, dbeta, dg fp32, dh0 fp32 or None), the reference's
    order (chunk.py:146).
    """
    dev = _require_device(q, k, v, g, beta, initial_state, do, dht)
    B, T, H, K = q.shape
    V = v.shape[-1]
    if torch.float16 in (q.dtype, k.dtype, v.dtype):
        # fp16 runs the fp32 kernels (see _f16_as_f32); gradients come back in the inputs' dtypes
        dts = (q.dtype, k.dtype, v.dtype, beta.dtype)
        dq, dk, dv, db, dg, dh0 = chunk_gated_delta_rule_bwd_native(
            q.float(), k.float(), v.float(), *_f16_as_f32(g, beta), scale, *_f16_as_f32(initial_state), do.float(),
            dht, cu_seqlens,
            use_qk_l2norm_in_kernel)
        return dq.to(dts[0]), dk.to(dts[1]), dv.to(dts[2]), db.to(dts[3]), dg, dh0
    qk_dt, v_dt = _code(q, "q"), _code(v, "v")
    if qk_dt == _lib.F8E4M3:
        raise NotImplementedError("the backward pass takes bf16 or fp32 q/k; fp8 q/k are forward-only")
    g_dt, b_dt = _code(g, "g"), _code(beta, "beta")
    q, k, v, g, beta = (x.contiguous() for x in (q, k, v, g, beta))
    do = do.to(v.dtype).contiguous()
    n_seqs, cu = 0, None
    if cu_seqlens is not None:
        cu = _prepare_cu_seqlens(cu_seqlens, dev, T)
        n_seqs = cu.numel() - 1
    N = n_seqs if cu is not None else B
    h0, h0_dt = None, _lib.F32
    if initial_state is not None:
        h0 = initial_state if initial_state.dtype in (torch.float32, torch.bfloat16) else initial_state.float()
        h0 = h0.contiguous()
        h0_dt = _code(h0, "initial_state")
    dht_ = dht.to(torch.float32).contiguous() if dht is not None else None
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dg = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    db = torch.empty_like(beta)
    dh0 = torch.empty(N, H, K, V, device=dev, dtype=torch.float32) if h0 is not None else None
    l2 = int(bool(use_qk_l2norm_in_kernel))
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_chunk_bwd_workspace_size(B, T, H, K, V, n_seqs, qk_dt, v_dt, l2)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    _lib.call("kairos_gdn_chunk_bwd", _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(h0), _ptr(do), _ptr(dht_),
              _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dg), _ptr(db), _ptr(dh0), _ptr(cu), n_seqs, B, T, H, K, V, qk_dt,
              v_dt, g_dt, b_dt, h0_dt, float(scale), l2, _ptr(ws), ws_bytes, _stream(dev))
    return dq, dk, dv, db, dg, dh0


class ChunkGatedDeltaRuleFunction(torch.autograd.Function):
    """Autograd wrapper (the reference's is chunk.py:149-213).

    forward saves the inputs; backward runs the native backward, which
    recomputes the forward's intermediates (the reference saves the normalised
    q, k and Ai, chunk.py:182, and recomputes w, u, h and v_new, chunk.py:84-101).
    """

    @staticmethod
    def forward(ctx, q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens=None,
                use_qk_l2norm_in_kernel=False, q_scale=None, k_scale=None):
        o, ht = chunk_gated_delta_rule_fwd(q, k, v, g, beta, scale, initial_state, output_final_state,
                                           cu_seqlens, use_qk_l2norm_in_kernel, q_scale, k_scale)
        ctx.save_for_backward(q, k, v, g, beta, initial_state, cu_seqlens)
        ctx.scale = scale
        ctx.use_qk_l2norm_in_kernel = use_qk_l2norm_in_kernel
        out_dtype = v.dtype if (_FP8 is not None and q.dtype == _FP8) else q.dtype
        return o.to(out_dtype), ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g, beta, initial_state, cu_seqlens = ctx.saved_tensors
        dq, dk, dv, db, dg, dh0 = chunk_gated_delta_rule_bwd_native(q, k, v, g, beta, ctx.scale, initial_state, do,
                                                                    dht, cu_seqlens, ctx.use_qk_l2norm_in_kernel)
        return dq.to(q), dk.to(k), dv.to(v), dg.to(g), db.to(beta), None, dh0, None, None, None, None, None


@torch.compiler.disable
def chunk_gated_delta_rule(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                           scale: float = None, initial_state: torch.Tensor = None, output_final_state: bool = False,
                           use_qk_l2norm_in_kernel: bool = False, cu_seqlens: torch.LongTensor | None = None,
                           **kwargs):
    r"""Chunked gated delta rule forward on MI355X.

    Same contract as the reference (chunk.py:217-323):
      q, k [B, T, H, K]; v [B, T, H, V]; g (log-space gates) and beta [B, T, H];
      initial_state [N, H, K, V]; cu_seqlens int64 [N+1] for packed variable
      length input (B must be 1).  Returns (o [B, T, H, V], final_state
      [N, H, K, V] fp32 or None).  ``scale`` defaults to K ** -0.5.
    Extension: q/k may be torch.float8_e4m3fn with per-head fp32 dequantisation
    scales passed as ``q_scale=`` / ``k_scale=`` (shape [H]); o then has v's dtype.
    fp16 inputs are accepted and computed by the fp32 kernels (o is returned in fp16).
    """
    if 'head_first' in kwargs:
        warnings.warn(
            "head_first is deprecated and will be removed in a future version. "
            "Please use head_first=False for now instead.",
        )
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
    return ChunkGatedDeltaRuleFunction.apply(
        q, k, v, g, beta, scale, initial_state, output_final_state, cu_seqlens, use_qk_l2norm_in_kernel,
        kwargs.get("q_scale"), kwargs.get("k_scale"))


# ---------------------------------------------------------------------------
# stages
# ---------------------------------------------------------------------------
def _stage_setup(ref: torch.Tensor, cu_seqlens, T):
    dev = ref.device
    n_seqs, cu = 0, None
    if cu_seqlens is not None:
        cu = _prepare_cu_seqlens(cu_seqlens, dev, T)
        n_seqs = cu.numel() - 1
    lib = _lib.load()
    ws_bytes = lib.kairos_gdn_stage_workspace_size(n_seqs)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    return dev, cu, n_seqs, ws, ws_bytes


def num_chunks_bound(B: int, T: int, n_seqs: int = 0) -> int:
    return int(_lib.load().kairos_gdn_num_chunks_bound(B, T, n_seqs))


def chunk_local_cumsum(g: torch.Tensor, chunk_size: int = CHUNK, reverse: bool = False, scale: float = None,
                       cu_seqlens=None, head_first: bool = False, output_dtype: torch.dtype | None = torch.float,
                       **kwargs) -> torch.Tensor:
    """Chunk-local prefix sum of scalar gates (fla ops/utils/cumsum.py:425-462, scalar form
    :247-279), fp32 out; the reference's arguments in its order.  Built: chunk_size 64, forward
    direction, no scale, [B, T, H] layout, fp32 output; anything else raises."""
    if chunk_size != CHUNK:
        raise ValueError("only chunk_size=64 is built")
    if reverse or scale is not None or head_first or output_dtype not in (None, torch.float32):
        raise NotImplementedError("chunk_local_cumsum: only reverse=False, scale=None, head_first=False and an fp32 "
                                  "output are built")
    if g.dim() != 3:
        raise NotImplementedError("chunk_local_cumsum: only scalar gates [B, T, H] are built")
    _require_device(g)
    B, T, H = g.shape
    g = g.contiguous()
    dev, cu, n_seqs, ws, wsb = _stage_setup(g, cu_seqlens, T)
    gc = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    _lib.call("kairos_gdn_chunk_local_cumsum", _ptr(g), _code(g, "g"), _ptr(gc), _ptr(cu), n_seqs, B, T, H,
              _ptr(ws), wsb, _stream(dev))
    return gc


def prepare_wy(k, v, g, beta, cu_seqlens=None, return_A: bool = False, k_scale=None):
    """Fused cumsum + scaled K.K^T + (I+A)^-1 + w/u (the first four reference stages).

    Returns (gc [B,T,H] fp32, w [B,T,H,K], uT [NCb,H,V,64], A, Ai); A (fp32) and
    Ai ([B,T,H,64], storage dtype) are None unless ``return_A``.
    """
    _require_device(k, v, g, beta)
    B, T, H, K = k.shape
    V = v.shape[-1]
    k, v, g, beta = (x.contiguous() for x in (k, v, g, beta))
    dev, cu, n_seqs, ws, wsb = _stage_setup(k, cu_seqlens, T)
    nc = num_chunks_bound(B, T, n_seqs)
    cdt = v.dtype
    gc = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    w = torch.empty(B, T, H, K, device=dev, dtype=cdt)
    uT = torch.empty(nc, H, V, CHUNK, device=dev, dtype=cdt)
    A = torch.zeros(B, T, H, CHUNK, device=dev, dtype=torch.float32) if return_A else None
    Ai = torch.zeros(B, T, H, CHUNK, device=dev, dtype=cdt) if return_A else None
    ks = k_scale.to(device=dev, dtype=torch.float32).contiguous() if k_scale is not None else None
    _lib.call("kairos_gdn_prepare_wy", _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(ks), _ptr(gc), _ptr(w),
              _ptr(uT), _ptr(A), _ptr(Ai), _ptr(cu), n_seqs, B, T, H, K, V, _code(k, "k"), _code(v, "v"),
              _code(g, "g"), _code(beta, "beta"), _ptr(ws), wsb, _stream(dev))
    return gc, w, uT, A, Ai


def fwd_h(k, w, uT, gc, initial_state=None, output_final_state=False, cu_seqlens=None, k_scale=None):
    """State recurrence (fla ops/common/chunk_delta_h.py:454-500).

    Returns (hT [NCb,H,V,K], vnT [NCb,H,V,64], final_state [N,H,K,V] fp32 or None).
    """
    _require_device(k, w, uT, gc, initial_state)
    B, T, H, K = k.shape
    V = uT.shape[2]
    dev, cu, n_seqs, ws, wsb = _stage_setup(k, cu_seqlens, T)
    nc = num_chunks_bound(B, T, n_seqs)
    N = n_seqs if cu is not None else B
    cdt = w.dtype
    hT = torch.empty(nc, H, V, K, device=dev, dtype=cdt)
    vnT = torch.empty(nc, H, V, CHUNK, device=dev, dtype=cdt)
    ht = torch.empty(N, H, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    h0 = initial_state.contiguous() if initial_state is not None else None
    h0_dt = _code(h0, "initial_state") if h0 is not None else _lib.F32
    ks = k_scale.to(device=dev, dtype=torch.float32).contiguous() if k_scale is not None else None
    _lib.call("kairos_gdn_fwd_h", _ptr(k.contiguous()), _ptr(ks), _ptr(w.contiguous()), _ptr(uT.contiguous()),
              _ptr(gc.contiguous()), _ptr(h0), _ptr(hT), _ptr(vnT), _ptr(ht), _ptr(cu), n_seqs, B, T, H, K, V,
              _code(k, "k"), _code(w, "w"), h0_dt, _ptr(ws), wsb, _stream(dev))
    return hT, vnT, ht


def fwd_o(q, k, hT, vnT, gc, scale=None, cu_seqlens=None, q_scale=None, k_scale=None):
    """Output stage (fla ops/common/chunk_o.py:498-535); o [B,T,H,V] in the storage dtype."""
    _require_device(q, k, hT, vnT, gc)
    B, T, H, K = q.shape
    V = hT.shape[2]
    if scale is None:
        scale = K ** -0.5
    dev, cu, n_seqs, ws, wsb = _stage_setup(q, cu_seqlens, T)
    o = torch.empty(B, T, H, V, device=dev, dtype=hT.dtype)
    qs = q_scale.to(device=dev, dtype=torch.float32).contiguous() if q_scale is not None else None
    ks = k_scale.to(device=dev, dtype=torch.float32).contiguous() if k_scale is not None else None
    _lib.call("kairos_gdn_fwd_o", _ptr(q.contiguous()), _ptr(k.contiguous()), _ptr(qs), _ptr(ks),
              _ptr(hT.contiguous()), _ptr(vnT.contiguous()), _ptr(gc.contiguous()), _ptr(o), float(scale),
              _ptr(cu), n_seqs, B, T, H, K, V, _code(q, "q"), _code(hT, "hT"), _ptr(ws), wsb, _stream(dev))
    return o


def _tokens_ws(ref, cu_seqlens, T, H, K, V, dtype):
    dev, cu, n_seqs, _, _ = _stage_setup(ref, cu_seqlens, T)
    B = ref.shape[0]
    nbytes = _lib.load().kairos_gdn_stage_tokens_workspace_size(B, T, H, K, V, n_seqs, _lib_dtype(dtype))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    return dev, cu, n_seqs, ws, nbytes


def _lib_dtype(dtype):
    return {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}[dtype]


def recompute_w_u_fwd(k, v, beta=None, A=None, g=None, cu_seqlens=None, *, g_raw=None, k_scale=None):
    """Fused cumsum + K.K^T + (I+A)^-1 + w/u with u in the reference's layout.

    The reference (wy_fast.py:213-248) takes A = (I+A)^-1 and the cumsummed g from
    earlier stages; this stage forms both itself from the raw log-space gates, which are
    passed as the keyword ``g_raw``.  A call in the reference's form (A or g given) raises
    instead of reading its arguments with another meaning.  Returns (gc [B,T,H] fp32,
    w [B,T,H,K], u [B,T,H,V]).
    """
    if A is not None or g is not None:
        raise NotImplementedError("recompute_w_u_fwd forms A and the cumsummed gates itself: pass the raw gates as "
                                  "g_raw= and no A / g")
    if beta is None or g_raw is None:
        raise TypeError("recompute_w_u_fwd needs beta and g_raw")
    g = g_raw
    _require_device(k, v, g, beta)
    B, T, H, K = k.shape
    V = v.shape[-1]
    k, v, g, beta = (x.contiguous() for x in (k, v, g, beta))
    dev, cu, n_seqs, ws, wsb = _tokens_ws(k, cu_seqlens, T, H, K, V, v.dtype)
    gc = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    w = torch.empty(B, T, H, K, device=dev, dtype=v.dtype)
    u = torch.empty(B, T, H, V, device=dev, dtype=v.dtype)
    ks = k_scale.to(device=dev, dtype=torch.float32).contiguous() if k_scale is not None else None
    _lib.call("kairos_gdn_prepare_wy_tokens", _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(ks), _ptr(gc), _ptr(w),
              _ptr(u), None, None, _ptr(cu), n_seqs, B, T, H, K, V, _code(k, "k"), _code(v, "v"), _code(g, "g"),
              _code(beta, "beta"), _ptr(ws), wsb, _stream(dev))
    return gc, w, u


def chunk_gated_delta_rule_fwd_h(k, w, u, g=None, gk=None, initial_state=None, output_final_state=False,
                                 chunk_size: int = CHUNK, save_new_value: bool = True, cu_seqlens=None, *,
                                 k_scale=None):
    """State recurrence in the reference's layouts and argument order
    (fla ops/common/chunk_delta_h.py:454-500).

    g is the chunk-local cumsum of the gates (fp32), as the reference passes it; per-key
    gates (gk) and chunk sizes other than 64 are not built and raise.  Returns
    (h [NCb,H,K,V], v_new [B,T,H,V] or None without save_new_value, final_state [N,H,K,V]
    fp32 or None); h's first NT rows (the real chunks, sequence-major) are the reference's
    h [B, NT, H, K, V] flattened, the rest zeros.
    """
    if gk is not None:
        raise NotImplementedError("chunk_gated_delta_rule_fwd_h: per-key gates (gk) are not built")
    if chunk_size != CHUNK:
        raise ValueError("only chunk_size=64 is built")
    if g is None:
        raise NotImplementedError("chunk_gated_delta_rule_fwd_h: the scalar gates g are required")
    _require_device(k, w, u, g, initial_state)
    B, T, H, K = k.shape
    V = u.shape[-1]
    dev, cu, n_seqs, ws, wsb = _tokens_ws(k, cu_seqlens, T, H, K, V, w.dtype)
    nc = num_chunks_bound(B, T, n_seqs)
    N = n_seqs if cu is not None else B
    h = torch.empty(nc, H, K, V, device=dev, dtype=w.dtype)
    v_new = torch.empty(B, T, H, V, device=dev, dtype=w.dtype)
    ht = torch.empty(N, H, K, V, device=dev, dtype=torch.float32) if output_final_state else None
    h0 = initial_state.contiguous() if initial_state is not None else None
    h0_dt = _code(h0, "initial_state") if h0 is not None else _lib.F32
    ks = k_scale.to(device=dev, dtype=torch.float32).contiguous() if k_scale is not None else None
    _lib.call("kairos_gdn_fwd_h_tokens", _ptr(k.contiguous()), _ptr(ks), _ptr(w.contiguous()), _ptr(u.contiguous()),
              _ptr(g.contiguous()), _ptr(h0), _ptr(h), _ptr(v_new), _ptr(ht), _ptr(cu), n_seqs, B, T, H, K, V,
              _code(k, "k"), _code(w, "w"), h0_dt, _ptr(ws), wsb, _stream(dev))
    return h, (v_new if save_new_value else None), ht


def chunk_fwd_o(q, k, v, h, g=None, g_gamma=None, scale=None, cu_seqlens=None, chunk_size: int = CHUNK, *,
                q_scale=None, k_scale=None):
    """Output stage in the reference's layouts and argument order (fla ops/common/chunk_o.py:498-535).

    v is v_new [B,T,H,V], h [NCb,H,K,V] as chunk_gated_delta_rule_fwd_h returns it, g the
    cumsummed gates; o [B,T,H,V] in v's dtype.  Per-head constant decays (g_gamma) and chunk
    sizes other than 64 are not built and raise.
    """
    if g_gamma is not None:
        raise NotImplementedError("chunk_fwd_o: g_gamma is not built")
    if chunk_size != CHUNK:
        raise ValueError("only chunk_size=64 is built")
    if g is None:
        raise NotImplementedError("chunk_fwd_o: the scalar gates g are required")
    _require_device(q, k, v, h, g)
    B, T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    dev, cu, n_seqs, ws, wsb = _tokens_ws(q, cu_seqlens, T, H, K, V, v.dtype)
    if h.shape[0] < num_chunks_bound(B, T, n_seqs):
        raise ValueError(f"h holds {h.shape[0]} chunks; {num_chunks_bound(B, T, n_seqs)} are expected")
    o = torch.empty(B, T, H, V, device=dev, dtype=v.dtype)
    qs = q_scale.to(device=dev, dtype=torch.float32).contiguous() if q_scale is not None else None
    ks = k_scale.to(device=dev, dtype=torch.float32).contiguous() if k_scale is not None else None
    _lib.call("kairos_gdn_fwd_o_tokens", _ptr(q.contiguous()), _ptr(k.contiguous()), _ptr(qs), _ptr(ks),
              _ptr(h.contiguous()), _ptr(v.contiguous()), _ptr(g.contiguous()), _ptr(o), float(scale), _ptr(cu),
              n_seqs, B, T, H, K, V, _code(q, "q"), _code(v, "v"), _ptr(ws), wsb, _stream(dev))
    return o


def l2norm_fwd(x: torch.Tensor, eps: float = 1e-6, output_dtype: torch.dtype | None = None):
    """Row L2 normalisation (fla modules/l2norm.py:157-196): returns (y, rstd) as the reference
    does, y in x's dtype, rstd fp32 of shape x.shape[:-1].  eps is fixed at 1e-6 and y keeps
    x's dtype; other values raise."""
    if eps != 1e-6:
        raise ValueError("only eps=1e-6 is built (the reference default)")
    if output_dtype not in (None, x.dtype):
        raise NotImplementedError("l2norm_fwd: the output keeps x's dtype")
    _require_device(x)
    x = x.contiguous()
    y = torch.empty_like(x)
    D = x.shape[-1]
    rstd = torch.empty(x.shape[:-1], device=x.device, dtype=torch.float32)
    _lib.call("kairos_gdn_l2norm_fwd", _ptr(x), _ptr(y), _ptr(rstd), _code(x, "x"), x.numel() // D, D,
              _stream(x.device))
    return y, rstd
