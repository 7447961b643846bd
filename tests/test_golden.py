"""Golden fixtures (tests/golden/gdn_golden.npz, written by tests/golden/make_golden.py).

The expected outputs are the fp64 token-by-token recurrence, a code path that
shares nothing with the chunked restatement or the HIP kernels.  The CPU tests
check that the fixtures still match the recurrence and that the chunked oracle
reaches them within the north-star tolerances; the GPU test runs the HIP path
(through the C ABI) on the same inputs against the same expected outputs.

Tolerances (relative L2, fla's get_err_ratio): bf16 o <= 1e-2, final_state <= 5e-3;
fp32 both <= 1e-4.
"""
import os
import sys

import numpy as np
import pytest

from oracle import gdn_oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402

TOL = {"bf16": dict(o=1e-2, ht=5e-3), "fp32": dict(o=1e-4, ht=1e-4)}
CASES = make_golden.load()


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_matches_recurrence(name):
    """The stored outputs are the fp64 recurrence of the stored inputs (fixture integrity)."""
    c = CASES[name]
    o, ht = O.naive_recurrent(c["q"], c["k"], c["v"], c["g"], c["beta"], initial_state=c["h0"],
                              cu_seqlens=c["cu"], dtype="fp64")
    np.testing.assert_allclose(c["o"], o, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(c["ht"], ht, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", sorted(CASES))
def test_chunked_oracle_against_fixture(name):
    c = CASES[name]
    dt = c["dtype"]
    o, ht = O.chunk_gated_delta_rule(c["q"], c["k"], c["v"], c["g"], c["beta"], initial_state=c["h0"],
                                     output_final_state=True, cu_seqlens=c["cu"], dtype=dt)
    eo, eh = O.rel_l2(o, c["o"]), O.rel_l2(ht, c["ht"])
    assert eo < TOL[dt]["o"], eo
    assert eh < TOL[dt]["ht"], eh


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_path_against_fixture(name):
    import torch
    import kairos_gdn

    c = CASES[name]
    dt = c["dtype"]
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    print(f"golden {name}: q{c['q'].shape} v{c['v'].shape} {dt} cu={c['cu']}", flush=True)

    def dev(a, t):
        return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(t)

    cu = torch.tensor(c["cu"], dtype=torch.int64, device="cuda") if c["cu"] is not None else None
    o, ht = kairos_gdn.chunk_gated_delta_rule(
        dev(c["q"], tdt), dev(c["k"], tdt), dev(c["v"], tdt), dev(c["g"], torch.float32), dev(c["beta"], tdt),
        scale=c["scale"], initial_state=dev(c["h0"], torch.float32), output_final_state=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert o.dtype == tdt and tuple(o.shape) == c["o"].shape
    eo = O.rel_l2(o.float().cpu().numpy(), c["o"])
    eh = O.rel_l2(ht.float().cpu().numpy(), c["ht"])
    print(f"    rel-L2 o={eo:.3e} ht={eh:.3e}", flush=True)
    assert eo < TOL[dt]["o"]
    assert eh < TOL[dt]["ht"]
