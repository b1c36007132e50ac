"""The C-ABI library loads and exports every symbol include/vflash_amd.h declares.

CPU-only: no entry point that launches a kernel is called; argument checks
that fail before any launch are exercised (no work is enqueued on EINVAL).
"""

import ctypes
import re
from pathlib import Path

import pytest

from vflash_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "vflash_amd.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(vflash_\w+)\s*\(", text, re.M)))


def test_header_declares_the_path():
    names = declared()
    for must in (
        "vflash_quantize_rows_e4m3",
        "vflash_fp8_linear",
        "vflash_fp8_linear_planes",
        "vflash_gelu_quantize_rows_e4m3",
        "vflash_requant_rows_e4m3",
        "vflash_fp8_linear_gate_residual",
        "vflash_lora_down",
        "vflash_fp8_linear_lora",
        "vflash_fp8_linear_lora_branches",
        "vflash_fp8_linear_lora_gate_residual",
        "vflash_fp8_linear_swiglu_lora",
        "vflash_nvfp4_linear",
    ):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.library()
    for name in declared():
        assert hasattr(lib, name), name
    assert set(declared()) == set(_lib.SIGNATURES)


def test_status_strings_and_version():
    lib = _lib.library()
    assert lib.vflash_abi_version() == _lib.ABI_VERSION == 4
    assert lib.vflash_status_string(_lib.VFLASH_EINVAL) == b"argument outside the declared contract"
    assert lib.vflash_swiglu_parts(28672) == 112 and lib.vflash_swiglu_parts(256) == 1


@pytest.mark.parametrize(
    "args",
    [
        # null operands, k % 16, n % 16, lda < k: rejected before any launch
        (None, None, 64, None, None, 64, 1, 16, 64, None, None, 16, None),
        (16, 16, 64, 16, 16, 64, 1, 16, 24, None, 16, 16, None),
        (16, 16, 64, 16, 16, 64, 1, 24, 64, None, 16, 24, None),
        (16, 16, 32, 16, 16, 64, 1, 16, 64, None, 16, 16, None),
    ],
)
def test_contract_violations_return_einval_without_launching(args):
    lib = _lib.library()
    conv = [ctypes.c_void_p(a) if i in (0, 1, 3, 4, 9, 10, 12) and a is not None else a
            for i, a in enumerate(args)]
    assert lib.vflash_fp8_linear(*conv) == _lib.VFLASH_EINVAL


def test_nvfp4_and_lora_contracts():
    lib = _lib.library()
    p = ctypes.c_void_p(256)
    # n not a multiple of 128
    assert lib.vflash_nvfp4_linear(p, p, 64, p, p, p, 1, 64, 64, None, p, 64, None) == -1
    # rank 0 or past 512, and a t row stride below ceil16(rank) or not a multiple of 8
    assert lib.vflash_lora_down(p, 4, 64, 64, p, 0, p, 16, None) == -1
    assert lib.vflash_lora_down(p, 4, 64, 64, p, 513, p, 528, None) == -1
    assert lib.vflash_lora_down(p, 4, 64, 64, p, 20, p, 24, None) == -1
    assert lib.vflash_lora_down(p, 4, 64, 64, p, 20, p, 36, None) == -1
    assert lib.vflash_quantize_rows_lora_e4m3(p, 4, 64, 64, p, p, 16, p, 20, p, 24, None) == -1


def _gemm_head(p):
    return [p, p, 64, p, p, 64, 16, 96, 64, None]


def test_adapter_entry_contracts():
    lib = _lib.library()
    p = ctypes.c_void_p(256)
    one = (ctypes.c_float * 3)(1.0, 1.0, 1.0)
    # rank 0 and 129; ldb not a multiple of 8; ldt below the rank
    for rank, ldt, ldb in ((0, 16, 16), (129, 136, 136), (16, 16, 20), (16, 8, 16)):
        assert lib.vflash_fp8_linear_lora(*_gemm_head(p), p, ldt, p, ldb, rank, 1.0, 1.0, p, 96,
                                          None) == -1
    # branches: 4 branches, a branch width that is not a multiple of 32 (n 96 / 3 = 32 is one),
    # t_branch below the rank, ldt too short for the last branch
    assert lib.vflash_fp8_linear_lora_branches(*_gemm_head(p), p, 64, 16, p, 16, 16, 4, one, 1.0,
                                               p, 96, 0, 0, None) == -1
    head = _gemm_head(p)
    head[7] = 144  # n 144: branches of 48 columns
    assert lib.vflash_fp8_linear_lora_branches(*head, p, 64, 16, p, 16, 16, 3, one, 1.0, p, 144,
                                               0, 0, None) == -1
    assert lib.vflash_fp8_linear_lora_branches(*_gemm_head(p), p, 64, 8, p, 16, 16, 3, one, 1.0,
                                               p, 96, 0, 0, None) == -1
    assert lib.vflash_fp8_linear_lora_branches(*_gemm_head(p), p, 40, 16, p, 16, 16, 3, one, 1.0,
                                               p, 96, 0, 0, None) == -1
    # no scales array; overlapping planes
    assert lib.vflash_fp8_linear_lora_branches(*_gemm_head(p), p, 48, 16, p, 16, 16, 3, None, 1.0,
                                               p, 96, 0, 0, None) == -1
    assert lib.vflash_fp8_linear_lora_branches(*_gemm_head(p), p, 48, 16, p, 16, 16, 3, one, 1.0,
                                               p, 32, 32, 32, None) == -1
    # gate-residual with an adapter of rank 0; SwiGLU with n % 256
    assert lib.vflash_fp8_linear_lora_gate_residual(
        *_gemm_head(p), p, 96, 1, 16, None, 0, p, 96, p, 16, p, 16, 0, 1.0, 1.0, p, 96, None) == -1
    head = _gemm_head(p)
    head[7] = 384
    assert lib.vflash_fp8_linear_swiglu_lora(*head, p, 16, p, 16, 16, 1.0, 1.0, p, 192, p,
                                             None) == -1


def test_tiling_query_routes_shapes():
    # Host-side query of the GEMM tiling (no device work): the automatic choice,
    # and branch widths that exclude the 192-column tilings (96-column waves).
    lib = _lib.library()
    names = ("256x256", "256x192", "256x128", "128x192", "128x128", "128x128 one round", "128x64",
             "64x64")
    pick = lambda m, n, b=0: names[lib.vflash_fp8_gemm_tiling(m, n, 256, b)]
    assert pick(32760, 13824) == "256x256"
    assert pick(4096, 3072) == "256x192"
    assert pick(2100, 3712) == "128x128"
    assert pick(520, 4112) == "128x128 one round"
    assert pick(257, 528) == "64x64"
    assert pick(4096, 3072, 1024) != "256x192"
    assert 5120 % (int(pick(32760, 15360, 5120).split("x")[1].split()[0]) // 2) == 0
    assert lib.vflash_fp8_gemm_tiling(16, 16, 256, 48) == -1  # branch width not a multiple of 32
    assert lib.vflash_fp8_gemm_tiling(0, 16, 256, 0) == -1


def test_gate_residual_and_producer_contracts():
    lib = _lib.library()
    p = ctypes.c_void_p(256)
    # gate_tokens 0, and an index without rows: rejected before any launch
    assert lib.vflash_fp8_linear_gate_residual(p, p, 64, p, p, 64, 16, 64, 64, None, p, 64, 1, 0,
                                               None, 0, p, 64, p, 64, None) == -1
    assert lib.vflash_fp8_linear_gate_residual(p, p, 64, p, p, 64, 16, 64, 64, None, p, 64, 1, 16,
                                               p, 0, p, 64, p, 64, None) == -1
    # out aliasing the residual with another row stride
    assert lib.vflash_fp8_linear_gate_residual(p, p, 64, p, p, 64, 16, 64, 64, None, p, 64, 1, 16,
                                               None, 0, p, 64, p, 128, None) == -1
    # k not a multiple of 8, a NaN eps, a misaligned modulation row stride
    args = [p, 4, 12, 16, None, 1e-6, p, 16, p, 16, 4, None, 0, None, 0, p, p, 16, None]
    assert lib.vflash_rmsnorm_modulate_quantize_e4m3(*args) == -1
    args[2] = 16
    args[5] = float("nan")
    assert lib.vflash_rmsnorm_modulate_quantize_e4m3(*args) == -1
    args[5] = 1e-6
    args[7] = 20
    assert lib.vflash_rmsnorm_modulate_quantize_e4m3(*args) == -1


def test_no_process_wide_tuning_state_is_exported():
    # The GEMM tiling is chosen from each call's shape alone; no export can
    # change it for later calls.
    lib = _lib.library()
    assert not hasattr(lib, "vflash_set_gemm_tile")


def test_noalloc_entry_refuses_oversize_calls_before_touching_a_device():
    # m * swiglu_parts(n) beyond 16 MiB of fp32 maxima: VFLASH_ESCRATCH, no launch
    # (the check precedes the device's scratch address lookup, so it runs here).
    lib = _lib.library()
    p = ctypes.c_void_p(256)
    args = [p, p, 1024, p, p, 1024, 4194305, 256, 1024, None, p, 128, p, p, 4194320, None]
    assert lib.vflash_fp8_linear_swiglu_quantize_noalloc(*args) == _lib.VFLASH_ESCRATCH
    args[6], args[14] = 16, 16
    args[7] = 200  # n % 256: outside the contract
    assert lib.vflash_fp8_linear_swiglu_quantize_noalloc(*args) == _lib.VFLASH_EINVAL
    assert lib.vflash_status_string(_lib.VFLASH_ESCRATCH).startswith(b"the call needs more")
