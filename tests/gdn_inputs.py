"""Seeded synthetic inputs with the distributions of BASELINE.json's configs.

q, k ~ N(0, 1) then L2-normalised per head; v ~ N(0, 1); beta = sigmoid(N(0, 1));
g = -softplus(N(0, 1)) in fp32; h0 = 0.02 * N(0, 1) in fp32.  Values are
rounded to the storage dtype ("bf16" values are held in float32 arrays).
"""
from __future__ import annotations

import numpy as np

from oracle import gdn_oracle as O


def make_inputs(B, T, H, K, V, seed, dtype="bf16", n_states=None, h0_scale=0.02, beta_dtype=None):
    rng = np.random.default_rng(seed)
    f32 = np.float32

    def unit(shape):
        x = rng.standard_normal(shape, dtype=f32)
        x /= np.sqrt(np.sum(x * x, axis=-1, keepdims=True, dtype=f32))
        return x

    q = O.cast(unit((B, T, H, K)), dtype)
    k = O.cast(unit((B, T, H, K)), dtype)
    v = O.cast(rng.standard_normal((B, T, H, V), dtype=f32), dtype)
    beta = O.cast(1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H), dtype=f32))), beta_dtype or dtype)
    g = (-np.logaddexp(0.0, rng.standard_normal((B, T, H), dtype=f32))).astype(f32)
    N = B if n_states is None else n_states
    h0 = (h0_scale * rng.standard_normal((N, H, K, V), dtype=f32)).astype(f32) if h0_scale else None
    return dict(q=q, k=k, v=v, g=g, beta=beta, h0=h0)


def quantize_fp8(x):
    """Per-head e4m3 quantisation with scale = amax / 448."""
    amax = np.abs(x).max(axis=(0, 1, 3))                               # [H]
    scale = (amax / 448.0).astype(np.float32)
    codes = O.fp8_e4m3_quantize(x / scale[None, None, :, None])
    return codes, scale


def dequant_bf16(codes, scale):
    return O.to_bf16(O.fp8_e4m3_decode(codes) * scale[None, None, :, None])


# BASELINE.json configs (the streaming config 4 is built by its own test)
CONFIGS = {
    0: dict(B=1, T=512, H=4, K=64, V=64, dtype="fp32", zero_h0=True),
    1: dict(B=1, T=8192, H=20, K=128, V=128, dtype="bf16"),
    2: dict(B=1, T=32760, H=20, K=128, V=128, dtype="bf16"),
    3: dict(B=1, T=53040, H=20, K=128, V=128, dtype="bf16", cu=[0, 1560, 7800, 20280, 53040]),
}
