"""ctypes binding of libsoupk.so (C ABI: include/soupk.h).

The library is loaded once, from this package's directory.  There is no fallback: if the
library is missing or a call fails, the error is raised (the product path never routes through
a CPU or PyTorch re-implementation).  Tensor checks (device, dtype, contiguity, shape) are done
here, before any pointer crosses the boundary.
"""

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsoupk.so")
_lock = threading.Lock()
_lib = None

ABI_VERSION = 4
STATUS_SCRATCH_LIMIT = 20001          # SOUPK_STATUS_SCRATCH_LIMIT
LORA_SCRATCH_FLOATS = 4 << 20         # SOUPK_LORA_SCRATCH_FLOATS
DTYPE_F16 = 0
DTYPE_F32 = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> argument types (every entry point returns int status)
SIGNATURES = {
    "soupk_nf4_unpack": [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _p],
    "soupk_nf4_unpack_multi": [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _p],
    "soupk_nf4_unpack_multi_lora": [_i32, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _p, _p,
                                    _p, _p, _i64, _i32, _i32, _i32, _i32, _p],
    "soupk_index_inverse": [_p, _i64, _p, _i64, _p],
    "soupk_sum_partials": [_p, _i32, _i64, _i64, _p, _p],
    "soupk_rmsnorm_fwd": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _f32, _p],
    "soupk_rmsnorm_bwd": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p],
    "soupk_rope_pack_fwd": [_p, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32,
                            _i32, _i32, _i32, _p],
    "soupk_rope_pack_bwd": [_p, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _p],
    "soupk_swiglu_fwd": [_p, _p, _i64, _i64, _p],
    "soupk_swiglu_bwd_inplace": [_p, _p, _i64, _i64, _p],
    "soupk_head_stats_grad": [_p, _p, _p, _p, _p, _p, _f32, _i64, _i64, _p],
    "soupk_head_stats_grad_rows": [_p, _p, _p, _p, _i64, _p, _p, _p, _p, _f32, _i64, _i64, _p],
    "soupk_time_next_launch": [_p, _p],
    "soupk_bench_copy": [_p, _p, _i64, _p],
    "soupk_bench_empty": [_i32, _p],
    "soupk_bench_hold": [ctypes.c_double, _p],
    "soupk_attention_fwd": [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f32, _p],
    "soupk_attention_bwd": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32,
                            _i32, _f32, _p],
    "soupk_rope_pack_tokens": [_p, _p, _p, _i32, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32,
                               _i32, _p],
    "soupk_attention_varlen_fwd": [_p, _p, _i32, _p, _p, _i64, _i32, _i32, _i32, _f32, _p],
    "soupk_attention_varlen_bwd": [_p, _p, _i32, _p, _p, _p, _p, _p, _p, _i64, _i32, _p, _p,
                                   _i64, _i32, _i32, _i32, _f32, _p],
    "soupk_lora_stage": [_p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _p],
    "soupk_lora_fwd": [_p, _p, _f32, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _p],
    "soupk_lora_rope_fwd": [_p, _p, _f32, _p, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32, _i32,
                            _i32, _i32, _i32, _p],
    "soupk_lora_bwd_rows": [_p, _i64, _p, _i64, _p, _f32, _p, _p, _i64, _i32, _i32, _i32, _i32,
                            _p],
    "soupk_lora_bwd_params": [_p, _p, _p, _p, _i64, _p, _i64, _f32, _p, _i64, _p, _p, _p, _p,
                              _i64, _i32, _i32, _i32, _i32, _p],
    "soupk_lora_bwd_params_noalloc": [_p, _p, _p, _p, _i64, _p, _i64, _f32, _p, _p, _p, _p, _i64,
                                      _i32, _i32, _i32, _i32, _p],
    "soupk_gemm_tn": [_p, _i64, _p, _p, _p, _i64, _i32, _i32, _p],
    "soupk_init_device": [],
    "soupk_gemm_nn_nf4": [_p, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _i64,
                          _i32, _i32, _p],
    "soupk_gemm_tn_nf4": [_p, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _p, _i64,
                          _i32, _i32, _p],
    "soupk_gemm_tn_nf4_split": [_p, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _p,
                                _i64, _i32, _i32, _i32, _p, _i64, _p],
    "soupk_gemm_nn_nf4_split": [_p, _i64, _i32, _p, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _i64,
                                _i32, _i32, _i32, _p, _i64, _p],
    "soupk_gemm_lt": [_i32, _i32, _i64, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64,
                      _i32, _i32, _i32, _p, _i32, _p, _i64, _p],
    "soupk_gemm_lt_index": [_i32, _i32, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                            _i32, _i32, _i32, _i32, _i32, _i64],
    "soupk_layer_fwd": [_p, _p, _p],
    "soupk_layer_bwd": [_p, _p, _p],
}


class SoupkError(RuntimeError):
    """A soupk entry point rejected its arguments or its launch failed."""


def library_path():
    return _LIB_PATH


def load_library(path):
    """dlopen a soupk library at `path` and bind every entry point's signature."""
    if not os.path.exists(path):
        raise SoupkError(
            f"{path} is missing: build it with `python -m testt_amd.build_ext` "
            "(or __graft_entry__.build()) before using the kernels")
    handle = ctypes.CDLL(path)
    handle.soupk_abi_version.restype = ctypes.c_int
    handle.soupk_abi_version.argtypes = []
    version = handle.soupk_abi_version()
    if version != ABI_VERSION:
        raise SoupkError(f"{path}: ABI {version} != expected {ABI_VERSION}: rebuild")
    handle.soupk_status_string.restype = ctypes.c_char_p
    handle.soupk_status_string.argtypes = [ctypes.c_int]
    for name, args in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    return handle


def lib():
    """The package's library, loaded once (raises if it has not been built).  On a machine
    with a HIP device, the current device's per-device state is set up right away
    (soupk_init_device), so that no later call has to do it under graph capture."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            handle = load_library(_LIB_PATH)
            if torch.cuda.is_available():
                handle.soupk_init_device()   # (a failure here resurfaces at the call)
            _lib = handle
    return _lib


_entry = {}   # name -> the bound ctypes function of the package's library


def call(name, *args):
    """Invoke entry point `name`; raise SoupkError on a non-zero status."""
    fn = _entry.get(name)
    if fn is None:
        fn = _entry[name] = getattr(lib(), name)
    status = fn(*args)
    if status != 0:
        text = lib().soupk_status_string(status)
        text = text.decode() if text else "?"
        raise SoupkError(f"{name} failed with status {status}: {text}")


def ptr(tensor):
    """Device address of a tensor (None for None)."""
    return None if tensor is None else tensor.data_ptr()


# torch's raw current-stream query: the handle torch.cuda.current_stream(device).cuda_stream
# returns, without building a Stream object on every kernel call (about 1 us of host time).
# It is not public API, so the public form stands in wherever it is absent;
# tests/test_gpu_streams.py checks that both give the same handle.
_RAW_STREAM = getattr(getattr(torch, "_C", None), "_cuda_getCurrentRawStream", None)


def stream_of(tensor):
    """The current HIP stream of the tensor's device, as a raw handle."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(tensor.device.index)
    return public_stream_of(tensor)


def public_stream_of(tensor):
    """stream_of through torch's public API."""
    return torch.cuda.current_stream(tensor.device).cuda_stream


def require(tensor, name, dtype=None, ndim=None, device=None):
    """Kernel inputs must be contiguous HIP device tensors of the stated dtype."""
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor, got {type(tensor).__name__}")
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a HIP device tensor (got device {tensor.device}); "
                         "the soupk kernels have no CPU path")
    if device is not None and tensor.device != device:
        raise ValueError(f"{name} is on {tensor.device}, expected {device}")
    if dtype is not None and tensor.dtype is not dtype:
        raise TypeError(f"{name} must be {dtype}, got {tensor.dtype}")
    if ndim is not None and tensor.dim() != ndim:
        raise ValueError(f"{name} must have {ndim} dims, got shape {tuple(tensor.shape)}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return tensor
