"""Seeded random shapes through the whole op on the GPU against the CPU oracle.

Twenty-four cases drawn once from a fixed seed: head dims (64, 128, 256 with
value dims up to 256), batch or varlen layouts (empty and one-token sequences
included), in-op L2 norm on or off, initial state present or absent, final
state requested or not, bf16 or fp32, and for some cases a forced segment plan
(chunks per segment, so the segment scan's chains take every remainder) or a
forced pipeline cut of the K = 256 form.  Bars as in test_gpu_parity.py:
relative L2 of o <= 1e-2 and of the final state <= 5e-3 in bf16, 1e-4 in fp32.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
from gdn_inputs import make_inputs
import kairos_gdn

pytestmark = pytest.mark.gpu

TOL = {"bf16": dict(o=1e-2, ht=5e-3), "fp32": dict(o=1e-4, ht=1e-4)}
TDT = {"bf16": torch.bfloat16, "fp32": torch.float32}


def _cases(n=24, seed=20263):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        K = int(rng.choice([64, 128, 256]))
        V = int(rng.choice([64, 128] if K < 256 else [64, 128, 256]))
        dt = "fp32" if rng.random() < 0.15 else "bf16"
        H = int(rng.integers(1, 4))
        varlen = rng.random() < 0.4
        if varlen:
            n_seq = int(rng.integers(2, 6))
            lens = [int(x) for x in rng.integers(2, 400, n_seq)]
            lens[int(rng.integers(0, n_seq))] = int(rng.choice([0, 1]))   # an empty or one-token sequence
            B, T = 1, sum(lens)
            cu = [0] + [int(c) for c in np.cumsum(lens)]
        else:
            B, T, cu = int(rng.integers(1, 4)), int(rng.integers(1, 500)), None
        l2 = bool(rng.random() < 0.4) and dt == "bf16"
        with_h0 = bool(rng.random() < 0.7)
        out_final = bool(rng.random() < 0.8)
        seg = str(int(rng.choice([1, 2, 3, 5, 7]))) if (K <= 128 and dt == "bf16" and rng.random() < 0.5) else None
        pipe = str(int(rng.choice([2, 3, 5]))) if (K == 256 and cu is None and rng.random() < 0.5) else None
        out.append((f"r{i:02d}", dt, B, T, H, K, V, cu, l2, with_h0, out_final, seg, pipe))
    return out


CASES = _cases()


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu_ready():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    kairos_gdn._lib.load()


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_random_shape(case, monkeypatch):
    name, dt, B, T, H, K, V, cu, l2, with_h0, out_final, seg, pipe = case
    note(f"{name}: {dt} B={B} T={T} H={H} K={K} V={V} cu={cu} l2={l2} h0={with_h0} final={out_final} "
         f"seg_chunks={seg} pipe={pipe}")
    if seg is not None:
        monkeypatch.setenv("KAIROS_GDN_SEG_CHUNKS", seg)
    if pipe is not None:
        monkeypatch.setenv("KAIROS_GDN_WIDE_PIPE", pipe)
    n = len(cu) - 1 if cu is not None else None
    x = make_inputs(B, T, H, K, V, seed=int(name[1:]) + 31, dtype=dt, n_states=n)
    if l2:                                               # unnormalised rows for the in-op norm
        x["q"] = O.cast(x["q"] * 2.5, dt)
        x["k"] = O.cast(x["k"] * 0.4, dt)
    d = {kk: torch.from_numpy(np.ascontiguousarray(x[kk])).to("cuda").to(TDT[dt]) for kk in ("q", "k", "v", "beta")}
    d["g"] = torch.from_numpy(x["g"]).to("cuda")
    h0 = torch.from_numpy(x["h0"]).to("cuda") if with_h0 else None
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu is not None else None
    o, ht = kairos_gdn.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=h0,
                                              output_final_state=out_final, cu_seqlens=cu_t,
                                              use_qk_l2norm_in_kernel=l2)
    torch.cuda.synchronize()
    assert o.shape == (B, T, H, V) and o.dtype == TDT[dt]
    assert (ht is not None) == out_final
    o_r, ht_r = O.chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"],
                                         initial_state=x["h0"] if with_h0 else None, output_final_state=True,
                                         cu_seqlens=np.array(cu) if cu is not None else None,
                                         use_qk_l2norm_in_kernel=l2, dtype=dt)
    eo = O.rel_l2(o.float().cpu().numpy(), o_r)
    eh = O.rel_l2(ht.cpu().numpy(), ht_r) if out_final else 0.0
    note(f"    rel-L2 o={eo:.3e} ht={eh:.3e}")
    assert eo < TOL[dt]["o"]
    assert eh < TOL[dt]["ht"]
