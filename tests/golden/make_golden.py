"""Writes the golden fixtures of the chunked GatedDeltaNet forward (gdn_golden.npz).

Test infrastructure: the expected outputs come from the fp64 token-by-token
recurrence of the reference's semantics (fla ops/gated_delta_product/naive.py:23-35
with num_householder=1, ops/gated_delta_rule/fused_recurrent.py:88-119):

    S <- exp(g_t) S ;  v'_t = beta_t (v_t - S^T k_t) ;  S <- S + k_t v'_t^T ;  o_t = scale S^T q_t

which shares no code path with the chunked restatement or the HIP kernels.
Inputs follow BASELINE.json's distributions (q, k L2-normalised, v ~ N(0, 1),
beta = sigmoid(N(0, 1)), g = -softplus(N(0, 1)), h0 = 0.02 N(0, 1)), rounded to
bf16 where the case is a bf16 case (values stored as float32).

Cases (name: B, T, H, K, V, dtype, cu_seqlens):
  fp32_ragged    1, 130, 1, 64, 64, fp32, -             ragged tail (130 = 2*64 + 2)
  bf16_d128      1, 100, 1, 128, 128, bf16, -           the benchmark head dims
  bf16_varlen    1, 150, 2, 64, 64, bf16, [0, 70, 71, 150]    varlen with a 1-token sequence
  bf16_batch2    2, 80, 1, 64, 128, bf16, -             fixed-length batch of 2

Storage: bf16 inputs (h0 included: bf16 cases round it to bf16 values) as their
16-bit patterns (uint16), fp32 inputs as float32, expected outputs rounded from
fp64 to float32.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from oracle import gdn_oracle as O  # noqa: E402
from gdn_inputs import make_inputs  # noqa: E402

CASES = {
    "fp32_ragged": dict(B=1, T=130, H=1, K=64, V=64, dtype="fp32", cu=None, seed=101),
    "bf16_d128": dict(B=1, T=100, H=1, K=128, V=128, dtype="bf16", cu=None, seed=102),
    "bf16_varlen": dict(B=1, T=150, H=2, K=64, V=64, dtype="bf16", cu=[0, 70, 71, 150], seed=103),
    "bf16_batch2": dict(B=2, T=80, H=1, K=64, V=128, dtype="bf16", cu=None, seed=104),
}
PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gdn_golden.npz")


def load(path=PATH):
    """{case: dict(q, k, v, g, beta, h0 (float32 arrays), cu (int64 or None), o, ht, dtype, scale)}."""
    z = np.load(path)
    cases = {}
    for name, c in CASES.items():
        d = {}
        for key in ("q", "k", "v", "beta", "h0"):
            a = z[f"{name}/{key}"]
            d[key] = (a.astype(np.uint32) << 16).view(np.float32) if a.dtype == np.uint16 else a
        for key in ("g", "o", "ht"):
            d[key] = z[f"{name}/{key}"]
        cu = z[f"{name}/cu"]
        d["cu"] = cu if cu.size else None
        d["dtype"] = c["dtype"]
        d["scale"] = c["K"] ** -0.5
        cases[name] = d
    return cases


def build():
    arrays = {}
    for name, c in CASES.items():
        n_states = len(c["cu"]) - 1 if c["cu"] is not None else c["B"]
        x = make_inputs(c["B"], c["T"], c["H"], c["K"], c["V"], c["seed"], c["dtype"], n_states=n_states)
        if c["dtype"] == "bf16":
            x["h0"] = O.to_bf16(x["h0"])
        cu = np.asarray(c["cu"], np.int64) if c["cu"] is not None else None
        o, ht = O.naive_recurrent(x["q"], x["k"], x["v"], x["g"], x["beta"], initial_state=x["h0"],
                                  cu_seqlens=cu, dtype="fp64")
        for key in ("q", "k", "v", "beta", "h0"):
            a = x[key].astype(np.float32)
            arrays[f"{name}/{key}"] = (a.view(np.uint32) >> 16).astype(np.uint16) if c["dtype"] == "bf16" else a
        arrays[f"{name}/g"] = x["g"].astype(np.float32)
        arrays[f"{name}/o"] = o.astype(np.float32)
        arrays[f"{name}/ht"] = ht.astype(np.float32)
        arrays[f"{name}/cu"] = cu if cu is not None else np.zeros(0, np.int64)
    return arrays


if __name__ == "__main__":
    np.savez_compressed(PATH, **build())
    print(f"wrote {PATH} ({os.path.getsize(PATH)} bytes)")
