"""ctypes binding of `libvgo.so` (the C ABI declared in include/vgo.h).

The library is loaded after torch so that it binds to the HIP runtime torch
already mapped (both carry the SONAME libamdhip64.so.7).  Nothing here falls
back to a CPU implementation: a missing library or a CPU tensor is an error.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "libvgo.so"

VGO_OK = 0
VGO_EINVAL = -1
VGO_ELAUNCH = -2
VGO_EUNSUPPORTED = -3
VGO_EWORKSPACE = -4

VGO_F32, VGO_BF16, VGO_F16 = 0, 1, 2
DTYPE_CODE = {torch.float32: VGO_F32, torch.bfloat16: VGO_BF16, torch.float16: VGO_F16}

_c_i64 = ctypes.c_int64
_c_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_f32 = ctypes.c_float
_c_size = ctypes.c_size_t
_i64x3 = ctypes.c_int64 * 3


class AttnProblem(ctypes.Structure):
    """`vgo_attn_problem` of include/vgo.h."""

    _fields_ = [
        ("q", _c_p), ("k", _c_p), ("v", _c_p), ("log_mass", _c_p), ("out", _c_p),
        ("batch", _c_i64), ("heads", _c_i64), ("n_query", _c_i64), ("n_key", _c_i64),
        ("head_dim", _c_i64),
        ("q_stride", _i64x3), ("k_stride", _i64x3), ("v_stride", _i64x3), ("o_stride", _i64x3),
    ]


# name -> (restype, argtypes); every symbol declared in include/vgo.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "vgo_last_error": (ctypes.c_char_p, []),
    "vgo_abi_version": (_c_int, []),
    "vgo_mass_bias_attn_fwd": (_c_int, [
        _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _i64x3, _i64x3, _i64x3, _i64x3, _c_int, _c_p,
    ]),
    "vgo_mass_bias_attn_workspace": (_c_int, [
        _c_i64, _c_i64, _c_i64, _c_i64, _c_int, ctypes.POINTER(_c_size),
    ]),
    "vgo_mass_bias_attn_fwd_ws": (_c_int, [
        _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _i64x3, _i64x3, _i64x3, _i64x3, _c_int, _c_p, _c_size, _c_p,
    ]),
    "vgo_mass_bias_attn_fwd_static": (_c_int, [
        _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _i64x3, _i64x3, _i64x3, _i64x3, _c_int, _c_p,
    ]),
    "vgo_mass_bias_attn_pair_workspace": (_c_int, [
        ctypes.POINTER(AttnProblem), _c_int, _c_int, ctypes.POINTER(_c_size),
    ]),
    "vgo_mass_bias_attn_pair_fwd_ws": (_c_int, [
        ctypes.POINTER(AttnProblem), _c_int, _c_int, _c_p, _c_size, _c_p,
    ]),
    "vgo_attn_kernel_timing": (_c_int, [_c_int]),
    "vgo_attn_kernel_timing_read": (_c_int, [
        ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_i64), ctypes.POINTER(_c_i64),
    ]),
    "vgo_attn_kernel_clock_read": (_c_int, [
        ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
        ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_c_i64),
    ]),
    "vgo_top4_project": (_c_int, [
        _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_p,
    ]),
    "vgo_top4_project_ordered": (_c_int, [
        _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_p,
    ]),
    "vgo_top4_gather_probe": (_c_int, [
        _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p,
    ]),
    "vgo_normalize_rows": (_c_int, [
        _c_p, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_i64, _c_f32, _c_p, _c_i64, _c_int, _c_p,
    ]),
    "vgo_similarity_topk_workspace": (_c_int, [
        _c_i64, _c_i64, _c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_size),
    ]),
    "vgo_similarity_topk": (_c_int, [
        _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
        _c_i64, _c_int, _c_p, _c_size, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p,
    ]),
    "vgo_fastvggt_assemble": (_c_int, [
        _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p,
    ]),
    "vgo_fastvggt_assemble_workspace": (_c_int, [_c_i64, _c_i64, _c_i64, ctypes.POINTER(_c_size)]),
    "vgo_fastvggt_assemble_ws": (_c_int, [
        _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_size,
        _c_p,
    ]),
    "vgo_sparse_convex_assemble": (_c_int, [
        _c_p, _c_p, _c_p, _c_p, _c_p, _c_f32, _c_p, _c_i64, _c_i64, _c_f32, _c_p, _c_p, _c_p,
        _c_p, _c_p, _c_p, _c_p,
    ]),
    "vgo_csr_workspace": (_c_int, [_c_i64, _c_i64, ctypes.POINTER(_c_size)]),
    "vgo_csr_build": (_c_int, [_c_p, _c_i64, _c_i64, _c_p, _c_size, _c_p, _c_p, _c_p]),
    "vgo_segment_mass": (_c_int, [
        _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_f32, _c_p, _c_p, _c_p,
    ]),
    "vgo_compact": (_c_int, [
        _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_int, _c_p, _c_p, _c_i64, _c_p,
        _c_i64, _c_i64, _c_p, _c_p, _c_f32, _c_p, _c_i64, _c_i64, _c_int, _c_int, _c_p,
    ]),
    "vgo_compact_multi": (_c_int, [
        _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_int, _c_p, _c_p, _c_i64, _c_p,
        _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p, _c_f32, _c_p, _c_p, _c_p, _c_int, _c_p,
    ]),
    "vgo_qkv_epilogue": (_c_int, [
        _c_p, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p,
        _c_p, _c_f32, _c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_int, _c_p,
    ]),
    "vgo_restore_map": (_c_int, [
        _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p,
    ]),
    "vgo_convex_fit": (_c_int, [
        _c_p, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p, _c_p, _c_f32, _c_p, _c_p, _c_i64, _c_i64,
        _c_f32, _c_f32, _c_p, _c_p, _c_p,
    ]),
    "vgo_failed_rows": (_c_int, [_c_p, _c_p, _c_f32, _c_i64, _c_f32, _c_p, _c_p, _c_p]),
    "vgo_four_support_active_set": (_c_int, [_c_p, _c_p, _c_i64, _c_f32, _c_p, _c_p]),
    "vgo_four_support_projected_gradient": (_c_int, [_c_p, _c_p, _c_i64, _c_int, _c_p, _c_p]),
    "vgo_residual_layer_norm": (_c_int, [
        _c_p, _c_i64, _c_p, _c_i64, _c_int, _c_p, _c_p, _c_p, _c_f32, _c_i64, _c_i64, _c_p, _c_i64,
        _c_p, _c_i64, _c_int, _c_p, _c_i64, _c_p, _c_i64, _c_f32, _c_p,
    ]),
    "vgo_restore_residual_layer_norm": (_c_int, [
        _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p, _c_p, _c_p, _c_f32, _c_i64,
        _c_i64, _c_p, _c_i64, _c_p, _c_i64, _c_int, _c_p,
    ]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class ExtensionUnavailable(RuntimeError):
    """Raised when the HIP library is missing or cannot be loaded."""


def load() -> ctypes.CDLL:
    """Load `libvgo.so` once and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY_PATH.exists():
            raise ExtensionUnavailable(
                f"vgo HIP extension is unavailable: {LIBRARY_PATH} is not built "
                "(run __graft_entry__.build())")
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH))
        except OSError as error:
            raise ExtensionUnavailable(f"vgo HIP extension failed to load: {error}") from error
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    return load().vgo_last_error().decode(errors="replace")


def check(status: int) -> None:
    """Map a C status to the exception types the reference raises."""
    if status == VGO_OK:
        return
    message = last_error()
    if status == VGO_EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def require_gpu(*tensors: torch.Tensor) -> None:
    for tensor in tensors:
        if tensor is not None and not tensor.is_cuda:
            raise RuntimeError("vgo kernels run on the GPU only; got a CPU tensor")


def stream_of(tensor: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on the tensor's device."""
    return torch.cuda.current_stream(tensor.device).cuda_stream


def ptr(tensor: torch.Tensor | None) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def strides3(tensor: torch.Tensor) -> ctypes.Array:
    s = tensor.stride()
    return _i64x3(s[0], s[1], s[2])


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None
