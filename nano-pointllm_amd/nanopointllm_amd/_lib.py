"""ctypes binding of libw8a8_gfx950.so (include/w8a8_gfx950.h).

The library is loaded from this package directory.  There is no fallback:
every GPU entry point raises ``RuntimeError`` when the library is missing,
and non-zero status codes become ``RuntimeError``/``ValueError``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libw8a8_gfx950.so"
ABI_VERSION = 7

F32, F16, BF16, I32, I8 = 0, 1, 2, 3, 4
EPI_I32, EPI_DEQUANT, EPI_SILU_MUL, EPI_SILU_MUL_Q8 = 0, 1, 2, 3
EPI_REQUANT, EPI_DEQUANT_BF16_EXACT = 4, 5
ROWS_AS_IS, ROWS_INTERLEAVE_HALVES = 0, 1

OK = 0
ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_ALIGN, ERR_WORKSPACE, ERR_HIP = -1, -2, -3, -4, -5, -6
ERR_TOO_LARGE = -7
ERR_OVERLAP = -8
NOALLOC_SCRATCH_BYTES = 16 << 20

# Names of the GEMM tiles w8a8_gemm_tile_config returns, by code.
GEMM_TILE_NAMES = ("tiny-deep", "small-deep", "big-deep", "big", "w192", "w224", "w256",
                   "w256sq", "mid", "wd7x2", "t112x96", "t128x96")

_TORCH_TO_CODE = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.int32: I32,
    torch.int8: I8,
}

EXPORTED_SYMBOLS = (
    "w8a8_abi_version",
    "w8a8_status_string",
    "w8a8_last_hip_error",
    "w8a8_packed_bytes",
    "w8a8_workspace_bytes",
    "w8a8_gemm_tile_config",
    "w8a8_quant_rows",
    "w8a8_quant_rows_scaled",
    "w8a8_pack_rows",
    "w8a8_gemm_i32",
    "w8a8_linear",
    "w8a8_linear_noalloc",
    "w8a8_rmsnorm_linear",
    "w8a8_rmsnorm_linear_ss",
    "w8a8_linear_residual",
    "w8a8_linear_i8in_residual",
    "w8a8_linear_i8in",
    "w8a8_linear_packed",
    "w8a8_linear_i8in_requant",
    "w8a8_gateup_silu_mul",
    "w8a8_gateup_workspace_bytes",
    "w8a8_prologue_quant",
    "w8a8_requantize_i32",
    "w8a8_dequant_i32_bf16",
    "w8a8_dense_gemv",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

_SIGNATURES = {
    "w8a8_abi_version": (_int, []),
    "w8a8_status_string": (ctypes.c_char_p, [_int]),
    "w8a8_last_hip_error": (_int, []),
    "w8a8_packed_bytes": (_i64, [_i64, _i64]),
    "w8a8_workspace_bytes": (_i64, [_i64, _i64]),
    "w8a8_gemm_tile_config": (_int, [_i64, _i64, _i64]),
    "w8a8_quant_rows": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "w8a8_quant_rows_scaled": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _vp]),
    "w8a8_pack_rows": (_int, [_vp, _i64, _i64, _i64, _int, _vp, _vp]),
    "w8a8_gemm_i32": (_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "w8a8_linear": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _int, _vp, _int, _i64, _f32, _int,
                           _i64, _i64, _i64, _vp, _vp, _i64, _vp]),
    "w8a8_linear_noalloc": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _int, _vp, _int, _i64, _f32,
                                   _int, _i64, _i64, _i64, _vp, _vp]),
    "w8a8_rmsnorm_linear": (_int, [_vp, _int, _i64, _vp, _i64, _vp, _i64, _vp, _f32, _vp, _vp,
                                   _vp, _int, _vp, _int, _i64, _f32, _int, _i64, _i64, _i64,
                                   _vp, _vp, _i64, _vp, _i64, _vp]),
    "w8a8_rmsnorm_linear_ss": (_int, [_vp, _int, _i64, _vp, _i64, _vp, _f32, _vp, _vp, _vp,
                                      _int, _vp, _int, _i64, _f32, _int, _i64, _i64, _i64, _vp,
                                      _vp, _i64, _vp]),
    "w8a8_linear_residual": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _vp, _int, _i64, _vp, _i64,
                                    _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "w8a8_linear_i8in_residual": (_int, [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _int, _i64, _vp,
                                         _i64, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp]),
    "w8a8_linear_i8in": (_int, [_vp, _i64, _vp, _vp, _vp, _vp, _int, _vp, _int, _i64, _f32,
                                _int, _i64, _i64, _i64, _vp, _i64, _vp]),
    "w8a8_linear_packed": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _vp, _int, _i64, _f32, _int,
                                  _i64, _i64, _i64, _vp]),
    "w8a8_linear_i8in_requant": (_int, [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                        _i64, _vp, _i64, _vp]),
    "w8a8_gateup_silu_mul": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _vp, _vp, _int, _i64, _vp,
                                    _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    "w8a8_gateup_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "w8a8_prologue_quant": (_int, [_vp, _int, _i64, _vp, _i64, _vp, _i64, _vp, _int, _f32, _vp,
                                   _vp, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _vp]),
    "w8a8_requantize_i32": (_int, [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "w8a8_dequant_i32_bf16": (_int, [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    "w8a8_dense_gemv": (_int, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _int, _i64, _i64, _i64,
                               _vp]),
}


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is absent or stale."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"W8A8 HIP library not found at {p}; build it with "
                "`python -m nanopointllm_amd.build` (there is no CPU fallback)")
        lib = ctypes.CDLL(str(p))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if lib.w8a8_abi_version() != ABI_VERSION:
            raise RuntimeError("W8A8 HIP library ABI version mismatch; rebuild it")
        if path is None:
            _lib = lib
        return lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_TO_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype for the W8A8 kernels: {dtype}") from None


def check(status: int, what: str) -> None:
    if status == OK:
        return
    lib = load()
    msg = lib.w8a8_status_string(status).decode()
    if status == ERR_HIP:
        raise RuntimeError(f"{what}: {msg} (hipError {lib.w8a8_last_hip_error()})")
    raise ValueError(f"{what}: {msg} (status {status})")


def stream_handle(device: torch.device) -> int:
    """The raw ``hipStream_t`` of torch's current stream on ``device`` (the
    direct query: building a ``torch.cuda.Stream`` object per launch costs
    more host time than the launch itself at decode shapes)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(index)


def require_cuda(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one GPU: the kernels have no host path."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "the W8A8 path runs only on the GPU through libw8a8_gfx950.so; "
                f"got a {t.device} tensor")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all tensors must be on the same device")
    if device is None:
        raise ValueError("no tensor given")
    return device


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
