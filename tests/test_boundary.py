"""CPU tests of the drop-in boundary: the C ABI library, its argument checks, the
Python host mirror's validation (reference error behaviour) and the swap.

No kernel is launched here: every C-ABI call below fails validation before
any HIP call, and the Python calls fail before reaching the library.
"""
import ctypes
import os
import re
import sys
import types
import warnings

import pytest
import torch

import kairos_gdn
from kairos_gdn import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "kairos_gdn.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(kairos_gdn_\w+)\s*\(", text)))


def test_library_is_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    lib = _lib.load()
    assert lib.kairos_gdn_abi_version() == _lib.ABI_VERSION


def test_library_exports_every_header_symbol():
    names = header_functions()
    assert len(names) >= 10
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), f"{n} declared in kairos_gdn.h but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_num_chunks_bound():
    lib = _lib.load()
    assert lib.kairos_gdn_num_chunks_bound(1, 32760, 0) == 512
    assert lib.kairos_gdn_num_chunks_bound(8, 1560, 0) == 8 * 25
    # varlen bound covers {1560, 6240, 12480, 32760}: 25 + 98 + 195 + 512 = 830 chunks
    assert lib.kairos_gdn_num_chunks_bound(1, 53040, 4) >= 830


def test_workspace_size():
    """The fused bf16 path holds one record per (chunk, head) -- the bf16 chunk
    inverse Ai (64 x 64) and eight fp32 chunk vectors of 64 -- and, for
    multi-segment sequences, the per-segment [M | R] maps and segment states
    (bounded by the CU count, not by T); the in-kernel L2 norm needs nothing more;
    the staged fp32 K=128 path holds the reference's per-chunk intermediates."""
    lib = _lib.load()

    def ai(nchunks, H):
        return nchunks * H * (64 * 64 * 2 + 8 * 64 * 4)

    def seg_state(B, T, H, K, V):
        L = lib.kairos_gdn_segment_chunks(B, T, H, 0)
        nseg = -(-(-(-T // 64)) // L)
        return 0 if nseg == 1 else B * nseg * H * (K * K + 2 * K * V) * 4

    ws = lib.kairos_gdn_chunk_fwd_workspace_size
    a = ws(1, 8192, 20, 128, 128, 0, _lib.BF16, _lib.BF16, 0)
    b = ws(1, 32760, 20, 128, 128, 0, _lib.BF16, _lib.BF16, 0)
    c = ws(1, 32760, 20, 128, 128, 0, _lib.BF16, _lib.BF16, 1)
    assert a == ai(128, 20) + seg_state(1, 8192, 20, 128, 128)
    assert b == ai(512, 20) + seg_state(1, 32760, 20, 128, 128)
    assert c == b                                 # the fused path folds the norm into its kernels
    assert ws(8, 1560, 20, 128, 128, 0, _lib.BF16, _lib.BF16, 0) == ai(8 * 25, 20)   # one segment each
    staged = ws(1, 8192, 20, 128, 128, 0, _lib.F32, _lib.F32, 0)
    assert staged > 8192 * 20 * 128 * 4 * 3


FAKE = 0x100000  # aligned non-null address: never dereferenced, validation fails first


def chunk_fwd_rc(**over):
    args = dict(q=FAKE, k=FAKE, v=FAKE, g=FAKE, beta=FAKE, q_scale=None, k_scale=None, h0=None, o=FAKE, ht=None,
                cu=None, n_seqs=0, B=1, T=128, H=2, K=64, V=64, qk=_lib.BF16, vdt=_lib.BF16, gdt=_lib.F32,
                bdt=_lib.BF16, h0dt=_lib.F32, scale=0.125, l2=0, ws=FAKE, wsb=0, stream=None)
    args.update(over)
    lib = _lib.load()
    rc = lib.kairos_gdn_chunk_fwd(*args.values())
    return rc, lib.kairos_gdn_last_error().decode()


@pytest.mark.parametrize("over,code,msg", [
    (dict(B=0), _lib.EINVAL, "invalid shape"),
    (dict(K=512), _lib.EINVAL, "larger than 256"),
    (dict(K=96), _lib.EUNSUPPORTED, "not built"),
    (dict(K=256, V=520), _lib.EUNSUPPORTED, "multiple of 16"),
    (dict(K=256, V=2048), _lib.EUNSUPPORTED, "not built"),
    (dict(B=2, cu=FAKE, n_seqs=1), _lib.EINVAL, "batch size is expected to be 1"),
    (dict(cu=FAKE, n_seqs=0), _lib.EINVAL, "given together"),
    (dict(qk=_lib.F8E4M3), _lib.EINVAL, "q_scale"),
    (dict(qk=_lib.F32), _lib.EINVAL, "dtype mix"),
    (dict(gdt=_lib.F8E4M3), _lib.EINVAL, "fp32 or bf16"),
    (dict(q=None), _lib.EINVAL, "null tensor"),
    (dict(v=FAKE + 2), _lib.EINVAL, "16-byte aligned"),
    (dict(scale=float("nan")), _lib.EINVAL, "finite"),
    (dict(wsb=16), _lib.EWORKSPACE, "workspace"),
])
def test_c_abi_rejects_invalid_arguments(over, code, msg):
    rc, err = chunk_fwd_rc(**over)
    assert rc == code
    assert msg in err


def test_stage_abi_rejects_invalid_arguments():
    lib = _lib.load()
    rc = lib.kairos_gdn_l2norm_fwd(FAKE, FAKE, None, _lib.BF16, 10, 100, None)
    assert rc == _lib.EINVAL and b"multiple of 8" in lib.kairos_gdn_last_error()
    rc = lib.kairos_gdn_fwd_o(FAKE, FAKE, None, None, FAKE, FAKE, FAKE, FAKE, 0.1, None, 0, 1, 64, 1, 64, 64,
                              _lib.F8E4M3, _lib.BF16, None, 0, None)
    assert rc == _lib.EINVAL and b"q_scale" in lib.kairos_gdn_last_error()
    rc = lib.kairos_gdn_prepare_wy(FAKE, FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, None, None, FAKE, 3, 1, 200, 2,
                                   64, 64, _lib.BF16, _lib.BF16, _lib.F32, _lib.F32, None, 0, None)
    assert rc == _lib.EWORKSPACE


def test_reference_layout_stage_abi_workspace_and_errors():
    """The reference-layout stages size their workspace as stage map + uT + hT + vnT, and reject
    head dims that are not multiples of 64 and short workspaces before touching the device."""
    lib = _lib.load()
    B, T, H, K, V = 2, 130, 3, 128, 64
    nc = lib.kairos_gdn_num_chunks_bound(B, T, 0)
    al = lambda x: (x + 255) // 256 * 256
    want = 2 * al(nc * H * V * 64 * 2) + al(nc * H * K * V * 2)
    assert lib.kairos_gdn_stage_tokens_workspace_size(B, T, H, K, V, 0, _lib.BF16) == want
    n_seqs = 3
    nc_v = lib.kairos_gdn_num_chunks_bound(1, T, n_seqs)
    want_v = al(4 * (n_seqs + 1)) + 2 * al(nc_v * H * V * 64 * 4) + al(nc_v * H * K * V * 4)
    assert lib.kairos_gdn_stage_tokens_workspace_size(1, T, H, K, V, n_seqs, _lib.F32) == want_v
    assert lib.kairos_gdn_stage_tokens_workspace_size(1, T, H, K, V, 0, _lib.F8E4M3) == 0
    rc = lib.kairos_gdn_fwd_h_tokens(FAKE, None, FAKE, FAKE, FAKE, None, FAKE, FAKE, None, None, 0, 1, 64, 1, 96, 64,
                                     _lib.BF16, _lib.BF16, _lib.F32, FAKE, 1 << 30, None)
    assert rc == _lib.EINVAL and b"multiples of 64" in lib.kairos_gdn_last_error()
    rc = lib.kairos_gdn_fwd_o_tokens(FAKE, FAKE, None, None, FAKE, FAKE, FAKE, FAKE, 0.1, None, 0, 1, 64, 1, 64, 64,
                                     _lib.BF16, _lib.BF16, FAKE, 16, None)
    assert rc == _lib.EWORKSPACE and b"workspace" in lib.kairos_gdn_last_error()
    rc = lib.kairos_gdn_prepare_wy_tokens(FAKE, FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, None, None, None, 0, 1, 64, 1,
                                          64, 64, _lib.F32, _lib.BF16, _lib.F32, _lib.F32, FAKE, 1 << 30, None)
    assert rc == _lib.EINVAL and b"dtype mix" in lib.kairos_gdn_last_error()


# ---------------------------------------------------------------------------
# Python host mirror: the reference's checks and messages (chunk.py:292-310)
# ---------------------------------------------------------------------------
def cpu_inputs(B=1, T=16, H=2, K=64, V=64):
    q = torch.randn(B, T, H, K)
    return q, q.clone(), torch.randn(B, T, H, V), -torch.rand(B, T, H), torch.rand(B, T, H)


def test_varlen_requires_batch_one():
    q, k, v, g, b = cpu_inputs(B=2)
    with pytest.raises(ValueError, match="batch size is expected to be 1 rather than 2"):
        kairos_gdn.chunk_gated_delta_rule(q, k, v, g, b, cu_seqlens=torch.tensor([0, 8, 16]))


def test_varlen_initial_state_count():
    q, k, v, g, b = cpu_inputs()
    h0 = torch.zeros(3, 2, 64, 64)
    with pytest.raises(ValueError, match="i.e., 2 rather than 3"):
        kairos_gdn.chunk_gated_delta_rule(q, k, v, g, b, initial_state=h0, cu_seqlens=torch.tensor([0, 8, 16]))


def test_cu_seqlens_checked_again_after_in_place_edit():
    """The host check of cu_seqlens is cached per tensor and version: editing a reused buffer in place
    (cu[1] beyond T) is caught again instead of reaching the kernels."""
    from kairos_gdn import chunk as ch
    cu = torch.tensor([0, 8, 16])
    assert ch._prepare_cu_seqlens(cu, torch.device("cpu"), 16).tolist() == [0, 8, 16]
    ch._prepare_cu_seqlens(cu, torch.device("cpu"), 16)          # cached: same object, same version
    cu[1] = 40
    with pytest.raises(ValueError, match="non-decreasing"):
        ch._prepare_cu_seqlens(cu, torch.device("cpu"), 16)
    cu[1] = 8
    with pytest.raises(ValueError, match="end at T=20"):
        ch._prepare_cu_seqlens(cu, torch.device("cpu"), 20)


def test_cu_seqlens_made_under_inference_mode():
    """A tensor made under torch.inference_mode() has no version counter: the host check runs on every
    call instead of failing on the missing counter, and still catches a bad edit."""
    from kairos_gdn import chunk as ch
    with torch.inference_mode():
        cu = torch.tensor([0, 8, 16])
        assert ch._prepare_cu_seqlens(cu, torch.device("cpu"), 16).tolist() == [0, 8, 16]
        assert ch._prepare_cu_seqlens(cu, torch.device("cpu"), 16).tolist() == [0, 8, 16]
        cu[1] = 40
        with pytest.raises(ValueError, match="non-decreasing"):
            ch._prepare_cu_seqlens(cu, torch.device("cpu"), 16)
    cu2 = torch.tensor([0, 4, 16])                      # an ordinary tensor after it is still cached and checked
    assert ch._prepare_cu_seqlens(cu2, torch.device("cpu"), 16).tolist() == [0, 4, 16]


def test_head_first_warns_and_cpu_tensors_are_refused():
    q, k, v, g, b = cpu_inputs()
    with warnings.catch_warnings(record=True) as rec:
        warnings.simplefilter("always")
        with pytest.raises(RuntimeError, match="HIP device only"):
            kairos_gdn.chunk_gated_delta_rule(q, k, v, g, b, head_first=False)
    assert any("head_first is deprecated" in str(w.message) for w in rec)


def test_stages_refuse_cpu_tensors():
    with pytest.raises(RuntimeError, match="HIP device only"):
        kairos_gdn.l2norm_fwd(torch.randn(4, 64))
    with pytest.raises(RuntimeError, match="HIP device only"):
        kairos_gdn.chunk_local_cumsum(torch.randn(1, 64, 2))


def test_backward_refuses_cpu_tensors_and_fp8():
    q, k, v, g, b = cpu_inputs()
    with pytest.raises(RuntimeError, match="HIP device only"):
        kairos_gdn.chunk_gated_delta_rule_bwd_native(q, k, v, g, b, 0.125, None, torch.randn(1, 16, 2, 64), None)
    lib = _lib.load()
    x = 16
    rc = lib.kairos_gdn_chunk_bwd(x, x, x, x, x, None, x, None, x, x, x, x, x, None, None, 0, 1, 64, 2, 64, 64,
                                  _lib.F8E4M3, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, 0.125, 0, None, 0, None)
    assert rc == _lib.EUNSUPPORTED and b"fp8" in lib.kairos_gdn_last_error()
    rc = lib.kairos_gdn_chunk_bwd(x, x, x, x, x, None, x, None, x, x, x, x, x, None, None, 0, 1, 64, 2, 64, 48,
                                  _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, 0.125, 0, None, 0, None)
    assert rc == _lib.EUNSUPPORTED
    rc = lib.kairos_gdn_chunk_bwd(x, x, x, x, x, None, x, None, x, x, x, x, x, x, None, 0, 1, 64, 2, 64, 64,
                                  _lib.BF16, _lib.BF16, _lib.F32, _lib.BF16, _lib.F32, 0.125, 0, None, 0, None)
    assert rc == _lib.EINVAL and b"dh0" in lib.kairos_gdn_last_error()
    assert lib.kairos_gdn_chunk_bwd_workspace_size(1, 64, 2, 64, 64, 0, _lib.BF16, _lib.BF16, 0) > 0


# ---------------------------------------------------------------------------
# swap (kairos_engine_patch-style rebinding of the op name)
# ---------------------------------------------------------------------------
def test_swap_rebinds_and_restores(monkeypatch):
    def reference_op(*a, **k):
        return "reference"

    class ReferenceNorm:
        pass

    class ReferenceConv:
        pass
    layer = types.ModuleType("fla.layers.gated_deltanet")
    layer.chunk_gated_delta_rule = reference_op
    layer.fused_recurrent_gated_delta_rule = reference_op
    layer.FusedRMSNormGated = ReferenceNorm
    layer.ShortConvolution = ReferenceConv
    vendored = types.ModuleType("kairos.third_party.fla.ops.gated_delta_rule")
    vendored.chunk_gated_delta_rule = reference_op
    monkeypatch.setitem(sys.modules, "fla.layers.gated_deltanet", layer)
    monkeypatch.setitem(sys.modules, "kairos.third_party.fla.ops.gated_delta_rule", vendored)
    patched = kairos_gdn.swap.install()
    assert set(patched) == {"fla.layers.gated_deltanet.chunk_gated_delta_rule",
                            "fla.layers.gated_deltanet.fused_recurrent_gated_delta_rule",
                            "fla.layers.gated_deltanet.FusedRMSNormGated",
                            "fla.layers.gated_deltanet.ShortConvolution",
                            "kairos.third_party.fla.ops.gated_delta_rule.chunk_gated_delta_rule"}
    assert layer.chunk_gated_delta_rule is kairos_gdn.chunk_gated_delta_rule
    assert layer.fused_recurrent_gated_delta_rule is kairos_gdn.fused_recurrent_gated_delta_rule
    assert layer.FusedRMSNormGated is kairos_gdn.FusedRMSNormGated
    assert layer.ShortConvolution is kairos_gdn.ShortConvolution
    assert vendored.chunk_gated_delta_rule is kairos_gdn.chunk_gated_delta_rule
    assert kairos_gdn.swap.install() == patched                  # idempotent
    restored = kairos_gdn.swap.uninstall()
    assert set(restored) == set(patched)
    assert layer.chunk_gated_delta_rule is reference_op
    assert layer.FusedRMSNormGated is ReferenceNorm and layer.ShortConvolution is ReferenceConv
    patched = kairos_gdn.swap.install(names=("chunk_gated_delta_rule",))   # the op alone
    assert layer.FusedRMSNormGated is ReferenceNorm and layer.chunk_gated_delta_rule is kairos_gdn.chunk_gated_delta_rule
    kairos_gdn.swap.uninstall()


# ---------------------------------------------------------------------------
# the product never routes through the oracle
# ---------------------------------------------------------------------------
def test_product_does_not_import_oracle():
    pkg = os.path.join(ROOT, "kairos-sensenova_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), f
                assert "gdn_oracle" not in text, f
