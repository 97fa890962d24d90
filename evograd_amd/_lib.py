"""ctypes binding of libevograd_hip.so (declared in include/evograd_hip.h).

torch is imported before the library is opened: torch ships the HIP runtime
(soname libamdhip64.so.7) and the dynamic loader then resolves the library's
own dependency to that same, already loaded runtime, so torch's streams and
device pointers are valid on both sides.

There is no fallback. If the library is missing or a launch fails the call
raises; nothing is ever computed on the CPU instead.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (loads the HIP runtime first; see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libevograd_hip.so")

EG_F32, EG_F16, EG_BF16 = 0, 1, 2
ABI_VERSION = 4

_DTYPE_TAG = {
    torch.float32: EG_F32,
    torch.float16: EG_F16,
    torch.bfloat16: EG_BF16,
}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_size = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/evograd_hip.h one for one.
SIGNATURES: dict[str, tuple] = {
    "eg_abi_version": (_i32, []),
    "eg_last_error": (ctypes.c_char_p, []),
    "eg_time_kernel": (_i32, [_p, _p, _i32]),
    "eg_time_kernel_missed": (_i32, []),
    "eg_time_kernel_label": (ctypes.c_char_p, []),
    "eg_softmax_fwd": (_i32, [_p, _p, _i64, _i64, _i32, _p]),
    "eg_softmax_bwd": (_i32, [_p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_rmsnorm_fwd": (_i32, [_p, _p, _p, _p, _i64, _i64, _f32, _i32, _p]),
    "eg_rmsnorm_workspace_bytes": (_size, [_i64, _i64]),
    "eg_rmsnorm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_rmsnorm_bwd_noalloc": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_fused_add_rmsnorm_fwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i64, _f32, _i32, _p]),
    "eg_fused_add_rmsnorm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_layernorm_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _f32, _i32, _p]),
    "eg_layernorm_workspace_bytes": (_size, [_i64, _i64]),
    "eg_layernorm_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_swiglu_fwd": (_i32, [_p, _p, _p, _i64, _i32, _p]),
    "eg_swiglu_bwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _p]),
    "eg_rope": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p]),
    "eg_attn_fwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "eg_attn_gqa_fwd": (_i32, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "eg_attn_workspace_bytes": (_size, [_i64, _i64, _i64, _i64]),
    "eg_attn_gqa_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "eg_attn_gqa_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "eg_attn_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "eg_llama3_attn_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i64]),
    "eg_llama3_attn_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "eg_llama3_attn_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p]),
    "eg_cross_entropy_workspace_bytes": (_size, [_i64]),
    "eg_cross_entropy_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p]),
    "eg_cross_entropy_bwd": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p]),
    "eg_cross_entropy_mean": (_i32, [_p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_flce_workspace_bytes": (_size, [_i64, _i64, _i64, _i64, _i32]),
    "eg_flce_fwd": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _p]),
    "eg_scale_copy": (_i32, [_p, _i32, _p, _i32, _i64, _p, _i32, _p, _p]),
    "eg_gemm_workspace_bytes": (_size, [_i64, _i64, _i64, _i32]),
    "eg_gemm": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32,
                       _i32, _i32, _p, _size, _p]),
    "eg_split_heads": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p]),
    "eg_merge_heads": (_i32, [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _p]),
    "eg_split_qkv_heads": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i32, _i32, _i32, _p]),
    "eg_merge_qkv_heads": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i32, _i32, _i32, _p]),
    "eg_add": (_i32, [_p, _p, _p, _i64, _i32, _p]),
    "eg_rmsnorm_bwd_small": (_i32, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_layernorm_bwd_small": (_i32, [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p]),
    "eg_silu_mul": (_i32, [_p, _p, _p, _i64, _i32, _p]),
    "eg_probe_mfma_bf16": (_i32, [_p, _p, _i32, _i32, _p]),
    "eg_probe_mfma_mix": (_i32, [_i32, _p, _p, _i32, _i32, _p]),
    "eg_gemm_segmented": (_i32, [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _i32,
                                 _i32, _p, _p, _p, _p, _i32, _i32, _p, _size, _p]),
}

_lib = None
_lock = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    pass


def load():
    """Open the library once and attach the C signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m evograd_amd.build` "
                "(or __graft_entry__.build()) first"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.eg_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryMissing(
                f"{LIB_PATH} has ABI {version}, this module expects {ABI_VERSION}; rebuild"
            )
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise RuntimeError with eg_last_error() on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.eg_last_error()
        raise RuntimeError(f"{name} failed (rc={rc}): {msg.decode() if msg else ''}")


def query(name: str, *args):
    return getattr(load(), name)(*args)


def dtype_tag(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_TAG[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(name: str, *tensors: torch.Tensor) -> None:
    """The kernels take device pointers only; refuse anything else loudly."""
    dev = None
    for t in tensors:
        if not torch.is_tensor(t):
            raise TypeError(f"{name}: expected a tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{name}: tensors must be on a ROCm GPU (got {t.device}); "
                "this library has no CPU path"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{name}: tensors on different devices ({dev} vs {t.device})")
