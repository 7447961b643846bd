"""GPU parity of the backward pass (kairos_gdn_chunk_bwd) against the backward oracle.

Every case runs the HIP backward through the C ABI (via the autograd Function
or chunk_gated_delta_rule_bwd) and compares dq, dk, dv, dg, dbeta and dh0 with
oracle/gdn_oracle_bwd.py on the same inputs: relative L2 <= 1e-2 for bf16 (the
north-star tolerance of o), <= 1e-4 for fp32.
"""
import numpy as np
import pytest
import torch

import kairos_gdn
from oracle import gdn_oracle as O
from oracle import gdn_oracle_bwd as OB
from gdn_inputs import make_inputs

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dv", "dg", "dbeta", "dh0")


def note(msg):
    print(msg, flush=True)


def run_case(B, T, H, K, V, seed, dtype="bf16", cu=None, h0=True, dht=True, l2=False, heads=None, tol=None):
    N = len(cu) - 1 if cu else B
    x = make_inputs(B, T, H, K, V, seed=seed, dtype=dtype, n_states=N, h0_scale=0.02 if h0 else 0.0)
    rng = np.random.default_rng(seed + 7)
    if l2:                                   # unnormalised q, k: the op normalises them
        x["q"] = O.cast(x["q"] * rng.uniform(0.5, 3.0, x["q"].shape[:-1] + (1,)).astype(np.float32), dtype)
        x["k"] = O.cast(x["k"] * rng.uniform(0.5, 3.0, x["k"].shape[:-1] + (1,)).astype(np.float32), dtype)
    do = O.cast(rng.standard_normal((B, T, H, V)).astype(np.float32), dtype)
    dht_ = rng.standard_normal((N, H, K, V)).astype(np.float32) if dht else None
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dev = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)  # noqa: E731
    cu_t = torch.tensor(cu, dtype=torch.int64, device="cuda") if cu else None
    dq, dk, dv, db, dg, dh0 = kairos_gdn.chunk_gated_delta_rule_bwd_native(
        dev(x["q"], tdt), dev(x["k"], tdt), dev(x["v"], tdt), dev(x["g"], torch.float32), dev(x["beta"], tdt),
        K ** -0.5, dev(x["h0"], torch.float32) if h0 else None, dev(do, tdt),
        dev(dht_, torch.float32) if dht else None, cu_t, l2)
    torch.cuda.synchronize()
    got = [g_.float().cpu().numpy() if g_ is not None else None for g_ in (dq, dk, dv, dg, db, dh0)]
    sel = (lambda a: a[:, :, heads]) if heads is not None else (lambda a: a)
    sel_s = (lambda a: a[:, heads]) if heads is not None else (lambda a: a)
    ref = OB.chunk_gated_delta_rule_bwd(sel(x["q"]), sel(x["k"]), sel(x["v"]), sel(x["g"]), sel(x["beta"]), sel(do),
                                        dht=sel_s(dht_) if dht else None, initial_state=sel_s(x["h0"]) if h0 else None,
                                        use_qk_l2norm_in_kernel=l2, cu_seqlens=cu, dtype=dtype)
    tol = tol or (1e-2 if dtype == "bf16" else 1e-4)
    errs = {}
    for n, a, b in zip(NAMES, got, ref):
        if b is None:
            assert a is None, n
            continue
        a = sel_s(a) if n == "dh0" else sel(a)
        assert np.isfinite(a).all(), n
        errs[n] = O.rel_l2(a, b)
    note("    " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    assert all(e < tol for e in errs.values()), errs
    return errs


CASES = [
    ("fp32 K=V=64 ragged", dict(B=1, T=130, H=2, K=64, V=64, seed=1, dtype="fp32")),
    ("fp32 K=V=128 varlen", dict(B=1, T=200, H=2, K=128, V=128, seed=2, dtype="fp32", cu=[0, 1, 70, 200])),
    ("bf16 K=V=128 batch 2", dict(B=2, T=200, H=2, K=128, V=128, seed=3)),
    ("bf16 K=V=64 no states", dict(B=1, T=100, H=3, K=64, V=64, seed=4, h0=False, dht=False)),
    ("bf16 varlen empty and 1-token sequences", dict(B=1, T=330, H=2, K=128, V=128, seed=5, cu=[0, 1, 1, 70, 200, 330])),
    ("bf16 in-op L2 norm", dict(B=1, T=190, H=2, K=128, V=128, seed=6, l2=True)),
    ("bf16 K=256 V=512 (the Kairos layer's head dims)", dict(B=1, T=150, H=2, K=256, V=512, seed=7)),
    ("bf16 K=128 V=256", dict(B=1, T=129, H=2, K=128, V=256, seed=8)),
]


@pytest.mark.parametrize("name,c", CASES, ids=[c[0] for c in CASES])
def test_bwd_against_oracle(name, c):
    note(f"backward {name}: {c}")
    run_case(**c)


def _random_cases(n=12, seed=20264):
    """Seeded random shapes for the backward: head dims (64, 128, 256 with value dims up to 256; fp32 at
    most 128), batch or varlen layouts with an empty or one-token sequence, in-op L2 norm, initial state
    and final-state gradient present or absent, bf16 or fp32."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        K = int(rng.choice([64, 128, 256]))
        V = int(rng.choice([64, 128] if K < 256 else [64, 128, 256]))
        dtype = "fp32" if rng.random() < 0.2 else "bf16"
        if dtype == "fp32":                  # the fp32 backward is built for K, V <= 128
            K, V = min(K, 128), min(V, 128)
        H = int(rng.integers(1, 3))
        c = dict(T=0, H=H, K=K, V=V, seed=100 + i, dtype=dtype, h0=bool(rng.random() < 0.7),
                 dht=bool(rng.random() < 0.7), l2=bool(rng.random() < 0.4) and dtype == "bf16")
        if rng.random() < 0.4:
            n_seq = int(rng.integers(2, 5))
            lens = [int(x) for x in rng.integers(2, 250, n_seq)]
            lens[int(rng.integers(0, n_seq))] = int(rng.choice([0, 1]))
            c.update(B=1, T=sum(lens), cu=[0] + [int(x) for x in np.cumsum(lens)])
        else:
            c.update(B=int(rng.integers(1, 3)), T=int(rng.integers(1, 300)))
        out.append((f"b{i:02d}", c))
    return out


RANDOM_CASES = _random_cases()


@pytest.mark.parametrize("name,c", RANDOM_CASES, ids=[c[0] for c in RANDOM_CASES])
def test_bwd_random_shapes(name, c):
    note(f"backward random {name}: {c}")
    run_case(**c)


def test_bwd_config1_all_heads():
    """BASELINE config 1 shape (B=1, T=8192, H=20, dk=dv=128, bf16, h0) with final-state gradient, every head."""
    note("backward config 1: B=1 T=8192 H=20 K=V=128 bf16")
    run_case(1, 8192, 20, 128, 128, seed=20261)


def _full_size_all_heads(B, T, H, K, V, seed, l2):
    """Backward at a full clip length on every head (oracle over head groups in child processes)."""
    import oracle_pool
    x = make_inputs(B, T, H, K, V, seed=seed, dtype="bf16")
    rng = np.random.default_rng(seed + 7)
    if l2:                                   # unnormalised q, k: the op normalises them
        for n in ("q", "k"):
            x[n] = O.cast(x[n] * rng.uniform(0.5, 3.0, x[n].shape[:-1] + (1,)).astype(np.float32), "bf16")
    do = O.cast(rng.standard_normal((B, T, H, V)).astype(np.float32), "bf16")
    dht = rng.standard_normal((B, H, K, V)).astype(np.float32)
    bf = torch.bfloat16
    dev = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)  # noqa: E731
    dq, dk, dv, db, dg, dh0 = kairos_gdn.chunk_gated_delta_rule_bwd_native(
        dev(x["q"], bf), dev(x["k"], bf), dev(x["v"], bf), dev(x["g"], torch.float32), dev(x["beta"], bf),
        K ** -0.5, dev(x["h0"], torch.float32), dev(do, bf), dev(dht, torch.float32), None, l2)
    torch.cuda.synchronize()
    host = lambda t: t.float().cpu().numpy()  # noqa: E731
    grads = dict(dq=host(dq), dk=host(dk), dv=host(dv), dg=host(dg), dbeta=host(db), dh0=host(dh0))
    for n, a_ in grads.items():
        assert np.isfinite(a_).all(), n
    note("    HIP backward done; oracle on every head")
    errs = oracle_pool.backward_all_heads(x, do, dht, grads, "bf16", workers=8, group=2, log=note,
                                          use_qk_l2norm_in_kernel=l2)
    note("    " + " ".join(f"{n}={e:.2e}" for n, e in errs.items()))
    assert all(e < 1e-2 for e in errs.values()), errs


def test_bwd_config2_shape_full_size():
    """The headline shape (T=32760, H=20, dk=dv=128, bf16, h0 and dht): the backward's segment scan (12
    segments per head) on every head against the oracle."""
    note("backward config 2 shape: B=1 T=32760 H=20 K=V=128, all heads")
    _full_size_all_heads(1, 32760, 20, 128, 128, seed=20262, l2=False)


def test_bwd_model_shape_full_size():
    """The Kairos layer in training: T=32760, H=20, dk=256, dv=512, the in-op L2 norm on unnormalised
    q, k, h0 and dht, on every head against the oracle."""
    note("backward model shape: B=1 T=32760 H=20 K=256 V=512 l2, all heads")
    _full_size_all_heads(1, 32760, 20, 256, 512, seed=20272, l2=True)


def test_bwd_model_shape_varlen():
    """The Kairos layer's head dims (dk=256, dv=512) at a varlen batch with initial states and the L2 norm."""
    note("backward K=256 V=512 varlen [0, 500, 1100] H=2 l2")
    run_case(1, 1100, 2, 256, 512, seed=9, cu=[0, 500, 1100], l2=True)


@pytest.mark.parametrize("form", ["fused recompute, 64-column dh kernel, 8-wave dq kernel", "16-column dh kernel",
                                  "4-wave dq kernel", "stage recompute"])
def test_bwd_model_head_dims_dh_forms(form, monkeypatch):
    """dk=256: h and v_new recomputed by the fused forward kernel in its recompute mode (the default)
    and by prepare's u pass + fwd_h; the dh recurrence with 64 value columns per workgroup (the
    default: q^T and w^T per chunk, loader waves, the snapshot and dv2 stored from LDS) and with 16
    columns; and the dq / dk / dw / dg stage with eight waves owning K rows (the default) and with four
    owning tokens: all match the oracle on a batch of 2 with a ragged last chunk at dv=512, and a varlen
    batch at dv=256 whose sequences are empty, 1 token, a chunk exactly and several chunks with a
    ragged end."""
    if "16-column" in form:
        monkeypatch.setenv("KAIROS_GDN_BWD_DHU_WIDE", "0")
    if "4-wave" in form:
        monkeypatch.setenv("KAIROS_GDN_BWD_DQK_WIDE", "0")
    if "stage recompute" in form:
        monkeypatch.setenv("KAIROS_GDN_BWD_RC_WIDE", "0")
    note(f"backward {form}: B=2 T=200 H=2 K=256 V=512")
    run_case(2, 200, 2, 256, 512, seed=31)
    note(f"backward {form}: varlen [0, 0, 1, 65, 400] H=2 K=256 V=256")
    run_case(1, 400, 2, 256, 256, seed=32, cu=[0, 0, 1, 65, 400])


@pytest.mark.parametrize("waves", ["16", "8", "4"])
def test_bwd_wy_forms(waves, monkeypatch):
    """The WY backward and the dv_local stage with sixteen, eight and four waves per chunk (WY: groups
    of four waves, each group on its share of the column tiles; bf16 takes sixteen where one
    workgroup fills a CU's LDS and eight where two fit): every form matches the oracle at every head
    dim the backward takes, on ragged batches and on a varlen batch with an empty and a 1-token
    sequence."""
    monkeypatch.setenv("KAIROS_GDN_BWD_WY_WAVES", waves)
    monkeypatch.setenv("KAIROS_GDN_BWD_DVL_WAVES", waves)
    note(f"backward, {waves}-wave WY and dv_local: B=2 T=333 H=2 K=64 V=64")
    run_case(2, 333, 2, 64, 64, seed=51)
    note(f"backward, {waves}-wave WY and dv_local: varlen [0, 0, 1, 200, 450] H=2 K=128 V=192")
    run_case(1, 450, 2, 128, 192, seed=52, cu=[0, 0, 1, 200, 450])
    note(f"backward, {waves}-wave WY and dv_local: B=1 T=300 H=2 K=256 V=512 l2")
    run_case(1, 300, 2, 256, 512, seed=53, l2=True)


@pytest.mark.parametrize("form", ["8-wave dq kernel", "8-wave dq kernel, two block buffers", "4-wave dq kernel"])
def test_bwd_dq_forms_k128(form, monkeypatch):
    """dk=128: the dq / dk / dw / dg stage with eight waves owning K rows (the default for bf16 K >= 128;
    one buffer of value-block tiles, two workgroups per CU, or two buffers) and with four owning tokens
    all match the oracle, on a ragged batch of 2, a varlen batch with an empty and a 1-token sequence,
    and with the in-op L2 norm (whose backward of q the eight-wave kernel applies itself and the
    four-wave form leaves to a pass of its own)."""
    if "4-wave" in form:
        monkeypatch.setenv("KAIROS_GDN_BWD_DQK_WIDE", "0")
    if "two block buffers" in form:
        monkeypatch.setenv("KAIROS_GDN_BWD_DQK_BUFS", "2")
    note(f"backward {form}: B=2 T=333 H=2 K=V=128")
    run_case(2, 333, 2, 128, 128, seed=41)
    note(f"backward {form}: varlen [0, 0, 1, 200, 450] H=3 K=128 V=192")
    run_case(1, 450, 3, 128, 192, seed=42, cu=[0, 0, 1, 200, 450])
    note(f"backward {form}: B=1 T=300 H=2 K=V=128 l2 (the norm's backward of q in the dq kernel or after it)")
    run_case(1, 300, 2, 128, 128, seed=43, l2=True)


@pytest.mark.parametrize("path", ["serial", "segments of 3 chunks", "segments of 1 chunk",
                                  "16-column dh kernel", "serial, 16-column dh kernel"])
def test_bwd_segment_scan_paths(path, monkeypatch):
    """The backward's segment scan (forward segment maps, dh reverse scan over segments) and the
    sequence-long recurrences both match the oracle, with the dh recurrence in its all-columns form
    and in its 16-column form: fixed length with a ragged last chunk, and a varlen batch whose
    sequences are empty, 1 token, a chunk exactly, and several segments long."""
    if "16-column" in path:
        monkeypatch.setenv("KAIROS_GDN_BWD_DHU_WIDE", "0")
    if path.startswith("serial"):
        monkeypatch.setenv("KAIROS_GDN_BWD_SEG", "0")
    elif "segments" in path:
        monkeypatch.setenv("KAIROS_GDN_SEG_CHUNKS", "3" if "3" in path else "1")
    note(f"backward {path}: fixed B=2 T=700 H=3")
    run_case(2, 700, 3, 128, 128, seed=12)
    note(f"backward {path}: varlen [0, 0, 1, 65, 129, 129, 900] H=2 K=64")
    run_case(1, 900, 2, 64, 128, seed=13, cu=[0, 0, 1, 65, 129, 129, 900])


def test_autograd_matches_direct_call():
    """torch.autograd through chunk_gated_delta_rule gives the direct backward call's gradients bit for bit."""
    B, T, H, K, V = 1, 150, 2, 128, 128
    x = make_inputs(B, T, H, K, V, seed=11, dtype="bf16")
    dev = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dt)  # noqa: E731
    bf = torch.bfloat16
    leaves = dict(q=dev(x["q"], bf), k=dev(x["k"], bf), v=dev(x["v"], bf), g=dev(x["g"], torch.float32),
                  beta=dev(x["beta"], bf), h0=dev(x["h0"], torch.float32))
    for t in leaves.values():
        t.requires_grad_(True)
    o, ht = kairos_gdn.chunk_gated_delta_rule(leaves["q"], leaves["k"], leaves["v"], leaves["g"], leaves["beta"],
                                              initial_state=leaves["h0"], output_final_state=True)
    gen = torch.Generator().manual_seed(3)
    do = torch.randn(o.shape, generator=gen).to("cuda", bf)
    dht = torch.randn(ht.shape, generator=gen).to("cuda")
    torch.autograd.backward([o, ht], [do, dht])
    direct = kairos_gdn.chunk_gated_delta_rule_bwd_native(*(leaves[n].detach() for n in ("q", "k", "v", "g", "beta")),
                                                          K ** -0.5, leaves["h0"].detach(), do, dht)
    for n, d in zip(("q", "k", "v", "beta", "g", "h0"), direct):
        assert leaves[n].grad is not None and leaves[n].grad.dtype == leaves[n].dtype, n
        assert torch.equal(leaves[n].grad, d.to(leaves[n].dtype)), n


def test_fp16_autograd_matches_fp32_inputs():
    """fp16 q/k/v/beta through autograd: the fp32 kernels on the same values, gradients returned in
    fp16 (dg and dh0 fp32); equal to the fp32-input call up to the fp16 rounding of the outputs."""
    B, T, H, K, V = 1, 200, 2, 128, 128
    x = make_inputs(B, T, H, K, V, seed=21, dtype="fp32")
    f16 = lambda a: a.astype(np.float16).astype(np.float32)  # noqa: E731
    for n in ("q", "k", "v", "beta"):
        x[n] = f16(x[n])
    rng = np.random.default_rng(22)
    do = f16(rng.standard_normal((B, T, H, V)).astype(np.float32))
    grads = {}
    for dt in (torch.float16, torch.float32):
        t = {n: torch.from_numpy(x[n]).to("cuda", dt).requires_grad_() for n in ("q", "k", "v", "beta")}
        g = torch.from_numpy(x["g"]).to("cuda").requires_grad_()
        h0 = torch.from_numpy(x["h0"]).to("cuda").requires_grad_()
        o, ht = kairos_gdn.chunk_gated_delta_rule(t["q"], t["k"], t["v"], g, t["beta"], initial_state=h0,
                                                  output_final_state=True, use_qk_l2norm_in_kernel=True)
        assert o.dtype == dt
        (o.float() * torch.from_numpy(do).cuda()).sum().add_(ht.square().sum() * 0.01).backward()
        torch.cuda.synchronize()
        for n in ("q", "k", "v", "beta"):
            assert t[n].grad.dtype == dt, n
        grads[dt] = [t[n].grad.float().cpu().numpy() for n in ("q", "k", "v", "beta")] + \
            [g.grad.cpu().numpy(), h0.grad.cpu().numpy()]
    errs = [O.rel_l2(a, b) for a, b in zip(grads[torch.float16], grads[torch.float32])]
    note("    fp16 vs fp32 inputs: " + " ".join(f"{e:.2e}" for e in errs))
    assert all(np.isfinite(a).all() for a in grads[torch.float16])
    assert all(e < 2e-3 for e in errs), errs

