"""ctypes binding of libvflash_amd.so (the C-ABI in include/vflash_amd.h).

The library is loaded lazily on first use.  There is no fallback: a missing
library or a device other than gfx950 raises, so no caller can silently run
another arithmetic.
"""

from __future__ import annotations

import ctypes
from functools import cache
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().with_name("libvflash_amd.so")

VFLASH_OK = 0
VFLASH_EINVAL = -1
VFLASH_ELAUNCH = -2
VFLASH_ESCRATCH = -3
NOALLOC_SCRATCH_BYTES = 16 << 20
ABI_VERSION = 4

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

# Signatures of every exported entry point (argument types, return type).
SIGNATURES: dict[str, tuple[list, object]] = {
    "vflash_abi_version": ([], _I32),
    "vflash_status_string": ([_I32], ctypes.c_char_p),
    "vflash_quantize_rows_e4m3": ([_P, _I64, _I64, _I64, _P, _P, _I64, _P], _I32),
    "vflash_fp8_linear": ([_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P], _I32),
    "vflash_fp8_linear_planes": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _P],
        _I32,
    ),
    "vflash_gelu_quantize_rows_e4m3": ([_P, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P], _I32),
    "vflash_fp8_linear_swiglu": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _P],
        _I32,
    ),
    "vflash_swiglu_parts": ([_I64], _I64),
    "vflash_fp8_linear_swiglu_quantize_noalloc": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _I64, _P],
        _I32,
    ),
    "vflash_rmsnorm_modulate_quantize_e4m3": (
        [_P, _I64, _I64, _I64, _P, _F32, _P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P, _P,
         _I64, _P],
        _I32,
    ),
    "vflash_requant_rows_e4m3": ([_P, _I64, _I64, _I64, _P, _I64, _P, _P, _I64, _P], _I32),
    "vflash_fp8_linear_gate_residual": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _P, _I64,
         _P, _I64, _P],
        _I32,
    ),
    "vflash_fp8_linear_lora_gate_residual": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _P, _I64,
         _P, _I64, _P, _I64, _I64, _F32, _F32, _P, _I64, _P],
        _I32,
    ),
    "vflash_lora_down": ([_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P], _I32),
    "vflash_quantize_rows_lora_e4m3": (
        [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _P], _I32),
    "vflash_fp8_linear_lora": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _F32, _F32,
         _P, _I64, _P],
        _I32,
    ),
    "vflash_fp8_linear_lora_branches": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _I64, _I64,
         ctypes.POINTER(_F32), _F32, _P, _I64, _I64, _I64, _P],
        _I32,
    ),
    "vflash_fp8_linear_swiglu_lora": (
        [_P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _I64, _F32, _F32,
         _P, _I64, _P, _P],
        _I32,
    ),
    "vflash_fp8_gemm_tiling": ([_I64, _I64, _I64, _I64], _I32),
    "vflash_nvfp4_linear": (
        [_P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P],
        _I32,
    ),
    "vflash_nvfp4_quantize_rows": ([_P, _I32, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P], _I32),
    "vflash_nvfp4_w4a4_linear": (
        [_P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P],
        _I32,
    ),
}


class KernelError(RuntimeError):
    """The HIP runtime refused a launch."""


@cache
def library() -> ctypes.CDLL:
    if not LIBRARY.exists():
        raise RuntimeError(
            f"{LIBRARY.name} is not built; run `python -m vflash_amd.build` (hipcc, gfx950)"
        )
    lib = ctypes.CDLL(str(LIBRARY))
    for name, (args, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = restype
    if lib.vflash_abi_version() != ABI_VERSION:
        raise RuntimeError("libvflash_amd.so has an unexpected ABI version")
    return lib


def call(name: str, *args) -> None:
    """Invoke an entry point; map a negative status to an exception."""
    status = getattr(library(), name)(*args)
    if status == VFLASH_OK:
        return
    text = library().vflash_status_string(status).decode()
    if status in (VFLASH_EINVAL, VFLASH_ESCRATCH):
        raise ValueError(f"{name}: {text}")
    raise KernelError(f"{name}: {text}")


# The per-call host path matters for launch-bound shapes (a skinny linear's
# kernels take a few microseconds): device facts that cannot change during a
# process are cached, and the stream comes from torch's raw accessor, which
# returns the pointer without building a Stream object.


@cache
def _cuda_present() -> bool:
    return torch.cuda.is_available()


@cache
def _gfx950_index(index: int) -> bool:
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0] == "gfx950"


def _index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def is_gfx950(device: torch.device) -> bool:
    if device.type != "cuda" or not _cuda_present():
        return False
    return _gfx950_index(_index(device))


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """Address of the current HIP stream of ``device`` (what the C-ABI takes as ``stream``)."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(_index(device))
    return torch.cuda.current_stream(device).cuda_stream


def ptr(tensor: torch.Tensor | None) -> int | None:
    """Device address of a tensor's first element, or None (NULL) for an absent operand."""
    return None if tensor is None else tensor.data_ptr()
