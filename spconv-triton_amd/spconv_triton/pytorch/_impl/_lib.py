"""ctypes binding of ``libspconv_hip.so``, the gfx950 C-ABI library.

The symbols and argument meanings are those declared in ``include/spconv_hip.h``.
Every call passes raw device pointers of torch tensors and torch's current
HIP stream; the library never allocates, so workspaces come from torch's
caching allocator.

There is no fallback: if the library is missing, or a tensor is not on the
GPU, the call raises.  The library must bind to the same HIP runtime as
torch; the loader checks that only one ``libamdhip64`` is mapped.
"""

from __future__ import annotations

import ctypes
import functools
import os
from pathlib import Path

import torch

_LIB_DIR = Path(__file__).resolve().parents[2] / "_lib"
LIB_PATH = _LIB_DIR / "libspconv_hip.so"

SP_OK = 0
SP_ERR_INVALID_ARG = 1
SP_ERR_UNSUPPORTED = 2
SP_ERR_WORKSPACE = 3
SP_ERR_HIP = 4
SP_ERR_HASH_FULL = 5

SP_F16, SP_BF16, SP_F32, SP_F64 = 0, 1, 2, 3
SP_PAIR_SUBM, SP_PAIR_REGULAR, SP_PAIR_TRANSPOSE = 0, 1, 2

SP_BF16X3 = 4  # fp32 operands as split-bf16 parts (SPCONV_ALLOW_TF32)

_DTYPE_CODE = {
    torch.float16: SP_F16,
    torch.bfloat16: SP_BF16,
    torch.float32: SP_F32,
    torch.float64: SP_F64,
}


class SpconvHipError(RuntimeError):
    """A library call failed inside HIP (launch error, runtime failure)."""


class Geom(ctypes.Structure):
    """Mirror of ``sp_geom`` (include/spconv_hip.h)."""

    _fields_ = [
        ("ndim", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("batch_size", ctypes.c_int64),
        ("in_shape", ctypes.c_int64 * 4),
        ("out_shape", ctypes.c_int64 * 4),
        ("ksize", ctypes.c_int32 * 4),
        ("stride", ctypes.c_int32 * 4),
        ("padding", ctypes.c_int32 * 4),
        ("dilation", ctypes.c_int32 * 4),
    ]


def make_geom(mode, batch_size, in_shape, out_shape, ksize, stride, padding, dilation) -> Geom:
    g = Geom()
    g.ndim = len(in_shape)
    g.mode = mode
    g.batch_size = int(batch_size)
    for i in range(g.ndim):
        g.in_shape[i] = int(in_shape[i])
        g.out_shape[i] = int(out_shape[i])
        g.ksize[i] = int(ksize[i])
        g.stride[i] = int(stride[i])
        g.padding[i] = int(padding[i])
        g.dilation[i] = int(dilation[i])
    return g


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U32 = ctypes.c_uint32
_SZ = ctypes.c_size_t
_GP = ctypes.POINTER(Geom)

# name -> (restype, argtypes); must match include/spconv_hip.h
_SIGNATURES = {
    "sp_abi_version": (ctypes.c_int, []),
    "sp_version": (ctypes.c_int, []),
    "sp_arch": (ctypes.c_char_p, []),
    "sp_last_error": (ctypes.c_char_p, []),
    "sp_geom_key64": (ctypes.c_int, [_GP]),
    "sp_pairgen_workspace_size": (_SZ, [_GP, _I64]),
    "sp_pairgen_subm": (ctypes.c_int, [_GP, _P, _I64, _P, _P, _P, _P, _SZ, _P]),
    "sp_pairgen_subm_grid_cells": (_I64, [_GP, _I64]),
    "sp_pairgen_subm_grid": (ctypes.c_int, [_GP, _P, _I64, _P, _P, _P, _P, _P, _I64,
                                            ctypes.c_uint32, _P]),
    "sp_pairgen_conv_build": (ctypes.c_int, [_GP, _P, _I64, _P, _SZ, ctypes.POINTER(_I64),
                                             ctypes.POINTER(_I64), _P]),
    "sp_pairgen_conv_fill": (ctypes.c_int, [_GP, _P, _I64, _P, _SZ, _I64, _P, _P, _P, _P, _P]),
    "sp_mask_words": (ctypes.c_int, [_P, _I64, _I64, _P, _P]),
    "sp_mask_sort_workspace_size": (_SZ, [_I64, _I32]),
    "sp_mask_sort": (ctypes.c_int, [_P, _I64, _I32, _I32, _U32, _I32, _P, _P, _P, _SZ, _P]),
    "sp_sort_dropped_positions": (ctypes.c_int, [ctypes.POINTER(ctypes.c_uint64), _I32]),
    "sp_compact_workspace_size": (_SZ, [_I64, _I64]),
    "sp_compact_table": (ctypes.c_int, [_P, _I64, _I64, _P, _P, _P, _P, _I32, _P, _SZ, _P]),
    "sp_native_to_tables": (ctypes.c_int, [_P, _I64, _I64, _I32, _I64, _I64, _P, _P, _P]),
    "sp_conv_workspace_size": (_SZ, [_I64, _I64, _I64, _I32]),
    "sp_conv_packed_bytes": (_SZ, [_I64, _I64, _I64, _I32, _I32]),
    "sp_conv_pack_weight": (ctypes.c_int, [_P, _I32, _P, _I64, _I64, _I64, _I32, _I32, _P, _P]),
    "sp_conv_gemm_packed": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _I64, _I64, _I32, _I32, _P,
                                           _I64, _P, _P, _P, _I32, _P]),
    "sp_gather_plan_bytes": (_SZ, [_I64, _I64]),
    "sp_gather_plan_overflow": (ctypes.c_int, [_P, _SZ, _I64, _I64, _P, _P]),
    "sp_gather_plan_build": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _I32, _P, _SZ,
                                            ctypes.POINTER(_I64), _P]),
    "sp_conv_gemm_planned": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _I64, _I64, _I32, _I32, _P,
                                            _I64, _P, _SZ, _P, _I32, _P]),
    "sp_conv_gemm_ordered": (ctypes.c_int, [_P, _I32, _I64, _P, _I64, _I64, _I64, _I32, _I32, _P,
                                            _I64, _P, _P, _SZ, _I32, _P, _I32, _P, _I32, _P]),
    "sp_permute_table": (ctypes.c_int, [_P, _I64, _I64, _P, _P, _P, _P]),
    "sp_table_stats": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P]),
    "sp_conv_fwd": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I32, _I64, _I64, _P, _I64, _P,
                                   _P, _P, _P, _I32, _P, _SZ, _P]),
    "sp_conv_fwd_noalloc": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I32, _I64, _I64, _P, _I64,
                                           _P, _P, _P, _P, _I32, _P]),
    "sp_conv_dgrad": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I32, _I64, _I64, _P, _I64, _P,
                                     _P, _P, _P, _SZ, _P]),
    "sp_split_bf16x3": (ctypes.c_int, [_P, _I64, _I64, _I32, _P, _P]),
    "sp_wgrad_workspace_size": (_SZ, [_I64, _I64, _I64, _I64]),
    "sp_conv_wgrad": (ctypes.c_int, [_P, _I64, _P, _I64, _I32, _I64, _I64, _I64, _P, _P, _P,
                                     _I64, _P, _P, _SZ, _P]),
    "sp_maxpool_fwd": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I64, _I64, _P, _P]),
    "sp_maxpool_bwd": (ctypes.c_int, [_P, _P, _P, _I32, _I64, _I64, _P, _I64, _I64, _P, _P]),
    "sp_avgpool_fwd": (ctypes.c_int, [_P, _I32, _I64, _I64, _P, _I64, _I64, _P, _P, _P]),
    "sp_avgpool_bwd": (ctypes.c_int, [_P, _P, _I32, _I64, _I64, _P, _I64, _I64, _P, _P]),
    "sp_point2voxel_workspace_size": (_SZ, [_I64, _I64]),
    "sp_point2voxel": (ctypes.c_int, [_P, _I32, _I64, _I64, _I32, _P, _P, _P, _I32, _I64, _I32,
                                      _I32, _I32, _P, _P, _P, _P, ctypes.POINTER(_I64), _P, _SZ,
                                      _P]),
    "sp_hash_table_bytes": (_SZ, [_I64]),
    "sp_hash_workspace_size": (_SZ, [_I64, _I64]),
    "sp_hash_clear": (ctypes.c_int, [_P, _I64, _P]),
    "sp_hash_insert": (ctypes.c_int, [_P, _I64, _P, _I32, _P, _I32, _I64, _U32,
                                      ctypes.POINTER(_I64), _P, _SZ, _P]),
    "sp_hash_insert_existing": (ctypes.c_int, [_P, _I64, _P, _I32, _P, _I32, _I64, _U32, _P, _P,
                                               _SZ, _P]),
    "sp_hash_query": (ctypes.c_int, [_P, _I64, _P, _I32, _I32, _I64, _P, _P, _P]),
    "sp_hash_items": (ctypes.c_int, [_P, _I64, _I32, _I32, _I64, _P, _P, _I32, _P, _SZ, _P]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

#: SP_ABI_VERSION of include/spconv_hip.h that _SIGNATURES follows.
ABI_VERSION = 2


def _hip_runtimes_mapped() -> set[str]:
    try:
        with open("/proc/self/maps") as f:
            lines = f.read().splitlines()
    except OSError:
        return set()
    paths = set()
    for line in lines:
        parts = line.split()
        if parts and "libamdhip64" in parts[-1]:
            paths.add(os.path.realpath(parts[-1]))
    return paths


@functools.lru_cache(maxsize=None)
def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load the library (no GPU call is made by loading)."""
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: the HIP library is not built.  Build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (or `make -C "
            "spconv-triton_amd/csrc`).  spconv_triton has no CPU or Triton fallback."
        )
    lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.sp_abi_version() != ABI_VERSION:
        raise RuntimeError(
            f"{p} has C ABI revision {lib.sp_abi_version()}, these bindings expect "
            f"{ABI_VERSION} (SP_ABI_VERSION of include/spconv_hip.h): rebuild the library"
        )
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise RuntimeError(
            "two HIP runtimes are mapped into this process "
            f"({sorted(runtimes)}); libspconv_hip.so must share torch's libamdhip64"
        )
    return lib


def lib() -> ctypes.CDLL:
    return load_library()


def last_error() -> str:
    msg = lib().sp_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(rc: int, what: str) -> None:
    if rc == SP_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == SP_ERR_INVALID_ARG:
        raise ValueError(msg)
    if rc == SP_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise SpconvHipError(f"{msg} (status {rc})")


def ptr(t: torch.Tensor | None):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None or t.numel() == 0:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_of(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise NotImplementedError(f"dtype {dtype} is not supported by spconv_triton") from None


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise AssertionError("spconv_triton kernels need GPU tensors")
