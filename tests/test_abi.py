"""The C ABI (CPU only, no kernel launches): libsoupk.so loads, exports every entry point that
include/soupk.h declares with the ctypes signature the Python layer binds, and rejects invalid
arguments before touching the GPU."""

import ctypes
import os
import re

import pytest

from testt_amd import _ext

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "soupk.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return dict(re.findall(r"\b(?:int|const char\*)\s+(soupk_\w+)\s*\(([^)]*)\)", text))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_ext.library_path()):
        pytest.fail("libsoupk.so is not built: run `python -m testt_amd.build_ext`")
    return _ext.lib()


def test_header_and_binding_agree(lib):
    decls = declared()
    assert set(decls) == set(_ext.SIGNATURES) | {"soupk_abi_version", "soupk_status_string"}
    for name, params in decls.items():
        n = 0 if params.strip() in ("", "void") else params.count(",") + 1
        if name in _ext.SIGNATURES:
            assert len(_ext.SIGNATURES[name]) == n, name


def test_every_declared_symbol_is_exported(lib):
    handle = ctypes.CDLL(_ext.library_path())
    for name in declared():
        assert hasattr(handle, name), f"{name} missing from libsoupk.so"


def test_version_and_status_strings(lib):
    assert lib.soupk_abi_version() == _ext.ABI_VERSION
    assert lib.soupk_status_string(0) == b"success"
    assert b"invalid" in lib.soupk_status_string(1)


@pytest.mark.parametrize("name,args", [
    ("soupk_swiglu_fwd", (None, None, -1, 8, None)),
    ("soupk_swiglu_bwd_inplace", (None, None, 4, 8, None)),
    ("soupk_nf4_unpack", (None,) * 7 + (64, 63, 256, None)),
    ("soupk_nf4_unpack_multi", (9,) + (None,) * 8 + (64, 256, None)),      # more than 8 parts
    ("soupk_sum_partials", (None, 0, 8, 8, None, None)),
    ("soupk_sum_partials", (None, 17, 8, 8, None, None)),
    ("soupk_sum_partials", (None, 2, 4, 8, None, None)),                    # stride < n
    ("soupk_sum_partials", (None, 2, 8, 8, None, None)),                    # null pointers
    ("soupk_nf4_unpack_multi", (1,) + (None,) * 8 + (63, 256, None)),
    ("soupk_nf4_unpack_multi", (2,) + (None,) * 8 + (64, 256, None)),      # null arrays
    ("soupk_rmsnorm_fwd", (None,) * 9 + (4, 0, 0, 1e-6, None)),
    ("soupk_rmsnorm_bwd", (None,) * 9 + (-1, 0, 16, None)),
    ("soupk_rope_pack_fwd", (None,) * 3 + (7,) + (None,) * 7 + (1, 1, 1, 1, 1, 8, None)),
    ("soupk_rope_pack_bwd", (None,) * 7 + (1, 1, 1, 1, 1, 7, None)),
    ("soupk_head_stats_grad", (None,) * 6 + (1.0, 1, 0, None)),
    # gradient rows: map without buffer, a pitch of part of a chunk, a misaligned buffer
    ("soupk_head_stats_grad_rows", (32, 32, 16, None, 1, 32, 32, 32, None, 1.0, 1, 8, None)),
    ("soupk_head_stats_grad_rows", (32, 32, 16, 64, 1, 32, 32, 32, None, 1.0, 1, 7, None)),
    ("soupk_head_stats_grad_rows", (32, 32, 16, 40, 1, 32, 32, 32, None, 1.0, 1, 8, None)),
    ("soupk_head_stats_grad_rows", (32, 32, 16, 64, -1, 32, 32, 32, None, 1.0, 1, 8, None)),
    ("soupk_index_inverse", (None, -1, None, 4, None)),
    ("soupk_bench_copy", (None, None, 4096, None)),
    ("soupk_bench_copy", (16, 32, 24, None)),        # not a multiple of 16 bytes
    ("soupk_bench_copy", (16, 32, 0, None)),
    ("soupk_bench_empty", (0, None)),
    ("soupk_bench_hold", (-1.0, None)),
    ("soupk_bench_hold", (2.5e6, None)),               # beyond the 2 s cap
    ("soupk_bench_hold", (float("nan"), None)),
    # LoRA staging: a buffer short of 128*H + 32*(NQ + NV) halves, a rank other than 16
    ("soupk_lora_stage", (16, 32, 48, 64, 128, 128 * 256 + 32 * 256 - 1, 256, 128, 128, 16,
                          None)),
    ("soupk_lora_stage", (16, 32, 48, 64, 128, 1 << 20, 256, 128, 128, 8, None)),
    # the unpack with the LoRA staging: the same LoRA rules, checked before the NF4 parts
    ("soupk_nf4_unpack_multi_lora", (0,) + (None,) * 8 + (64, 256) +
     (16, 32, 48, 64, 128, 1 << 20, 256, 128, 128, 8, None)),
    ("soupk_nf4_unpack_multi_lora", (0,) + (None,) * 8 + (64, 256) +
     (16, 32, 48, 64, 128, 100, 256, 128, 128, 16, None)),
    ("soupk_nf4_unpack_multi_lora", (0,) + (None,) * 8 + (64, 256) +
     (16, 32, 48, 64, 136, 1 << 20, 256, 128, 128, 16, None)),            # misaligned staged
    # the LoRA forward fused with the RoPE pack: head dim other than 128, no position rows, a
    # rank other than 16, null pointers, a misaligned output
    ("soupk_lora_rope_fwd", (16, 32, 2.0, 48, 64, 80, 96, 112, 128, 4, 256, 2, 1, 64, 16, 1, 4,
                             None)),
    ("soupk_lora_rope_fwd", (16, 32, 2.0, 48, 64, 80, 96, 112, 128, 4, 256, 2, 1, 128, 16, 1, 0,
                             None)),
    ("soupk_lora_rope_fwd", (16, 32, 2.0, 48, 64, 80, 96, 112, 128, 4, 256, 2, 1, 128, 8, 1, 4,
                             None)),
    ("soupk_lora_rope_fwd", (None, 32, 2.0, 48, 64, 80, 96, 112, 128, 4, 256, 2, 1, 128, 16, 1,
                             4, None)),
    ("soupk_lora_rope_fwd", (16, 32, 2.0, 48, 64, 80, 96, 112, 136, 4, 256, 2, 1, 128, 16, 1, 4,
                             None)),
    # the NF4 input-gradient GEMM: W columns not a multiple of 128, a contraction not a
    # multiple of 64, no parts, a blocksize other than 64
    ("soupk_gemm_nn_nf4", (16, 256, 1) + (16,) * 7 + (64, 256, 16, 4, 100, 256, None)),
    ("soupk_gemm_nn_nf4", (16, 256, 1) + (16,) * 7 + (64, 256, 16, 4, 128, 100, None)),
    ("soupk_gemm_nn_nf4", (16, 256, 0) + (16,) * 7 + (64, 256, 16, 4, 128, 256, None)),
    ("soupk_gemm_nn_nf4", (16, 256, 1) + (16,) * 7 + (32, 256, 16, 4, 128, 256, None)),
])
def test_invalid_arguments_rejected_before_launch(lib, name, args):
    with pytest.raises(_ext.SoupkError, match="status 1"):
        _ext.call(name, *args)


@pytest.mark.parametrize("name,args", [
    ("soupk_swiglu_fwd", (None, None, 0, 8960, None)),
    ("soupk_nf4_unpack", (None,) * 7 + (0, 64, 256, None)),
    ("soupk_nf4_unpack_multi", (0,) + (None,) * 8 + (64, 256, None)),
    ("soupk_sum_partials", (None, 4, 0, 0, None, None)),
    ("soupk_head_stats_grad", (None,) * 6 + (1.0, 0, 151936, None)),
    ("soupk_head_stats_grad_rows", (None,) * 4 + (0,) + (None,) * 4 + (1.0, 0, 151936, None)),
    ("soupk_index_inverse", (None, 0, None, 0, None)),
])
def test_empty_work_is_a_no_op(lib, name, args):
    _ext.call(name, *args)


def _split_args(M=16, N=256, K=256, splits=2, ws=None, bias=None):
    """soupk_gemm_tn_nf4_split arguments for one NF4 part of N rows: host arrays of fake,
    16-byte aligned device addresses (the checks below reject before any launch)."""
    one = lambda: (ctypes.c_void_p * 1)(4096)
    keep = [one() for _ in range(6)] + [(ctypes.c_int32 * 1)(N)]
    ws = 2 * M * N if ws is None else ws
    args = (4096, K, 1, *[ctypes.addressof(a) for a in keep], 64, 256, bias, 8192, M, N, K,
            splits, 16384, ws, None)
    return keep, args


@pytest.mark.parametrize("kw", [
    dict(splits=0), dict(splits=33, K=64 * 40, ws=1 << 30), dict(splits=5),   # 4 K tiles
    dict(splits=2, ws=2 * 16 * 256 - 1), dict(bias=4100),
])
def test_split_gemm_rejects_bad_splits_workspace_and_bias(lib, kw):
    keep, args = _split_args(**kw)
    with pytest.raises(_ext.SoupkError, match="status 1"):
        _ext.call("soupk_gemm_tn_nf4_split", *args)


def test_split_gemm_workspace_counts_used_splits(lib):
    """K = 320 (5 tiles) cut 4 ways runs 2 tiles per split, so 3 splits are used and the
    workspace needs 3 * M * N floats: 3 M N - 1 is rejected; with M = 0 nothing runs."""
    keep, args = _split_args(K=320, splits=4, ws=3 * 16 * 256 - 1)
    with pytest.raises(_ext.SoupkError, match="status 1"):
        _ext.call("soupk_gemm_tn_nf4_split", *args)
    keep, args = _split_args(M=0, K=320, splits=4, ws=0)
    _ext.call("soupk_gemm_tn_nf4_split", *args)


def _nn_split_args(M=16, N=128, K=256, splits=2, ws=None):
    """soupk_gemm_nn_nf4_split arguments for one NF4 part of K rows and N columns (fake device
    addresses, as _split_args)."""
    one = lambda: (ctypes.c_void_p * 1)(4096)
    keep = [one() for _ in range(6)] + [(ctypes.c_int32 * 1)(K)]
    ws = 2 * M * N if ws is None else ws
    args = (4096, K, 1, *[ctypes.addressof(a) for a in keep], 64, 256, 8192, M, N, K, splits,
            16384, ws, None)
    return keep, args


@pytest.mark.parametrize("kw", [
    dict(splits=0), dict(splits=33, K=64 * 40, ws=1 << 30), dict(splits=5),   # 4 steps
    dict(splits=2, ws=2 * 16 * 128 - 1), dict(N=96)])
def test_nn_split_gemm_rejects_bad_splits_and_workspace(lib, kw):
    keep, args = _nn_split_args(**kw)
    with pytest.raises(_ext.SoupkError, match="status 1"):
        _ext.call("soupk_gemm_nn_nf4_split", *args)
    keep, args = _nn_split_args(M=0, K=384, splits=4, ws=0)   # 3 of 4 splits used; no rows
    _ext.call("soupk_gemm_nn_nf4_split", *args)


def test_noalloc_rejects_problems_beyond_its_scratch(lib):
    """soupk_lora_bwd_params_noalloc returns SOUPK_STATUS_SCRATCH_LIMIT, before any HIP call,
    for a problem whose partial sums exceed its static scratch (6785 rows at the Qwen2.5-1.5B
    shapes; 6784 fit)."""
    H, NQ, NV = 1536, 1536, 256
    need = -(-6785 // 128) * (32 * H + 16 * (NQ + NV))
    assert need > _ext.LORA_SCRATCH_FLOATS >= -(-6784 // 128) * (32 * H + 16 * (NQ + NV))
    with pytest.raises(_ext.SoupkError, match=f"status {_ext.STATUS_SCRATCH_LIMIT}: .*scratch"):
        _ext.call("soupk_lora_bwd_params_noalloc", 16, 16, 16, 16, NQ, 16, NV, 2.0,
                  *(16,) * 4, 6785, H, NQ, NV, 16, None)
