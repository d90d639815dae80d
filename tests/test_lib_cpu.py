"""CPU-only checks of the boundary: the C-ABI library loads and exports every
symbol ``include/spconv_hip.h`` declares, the ctypes signatures cover exactly
those symbols, host-only queries behave, and the Python package exposes the
reference's public API (names and constructor signatures pinned by the
reference's ``tests/data/golden_api.json``, extracted to ``tests/golden/api.json``).
No GPU work is launched here.
"""

import ctypes
import inspect
import json
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "spconv_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_functions():
    names = _declared_functions()
    assert "sp_conv_fwd" in names and "sp_pairgen_subm" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    from spconv_triton.pytorch._impl import _lib

    lib = _lib.load_library()
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared_functions():
        assert hasattr(raw, name), f"{name} declared in spconv_hip.h but not exported"
        assert hasattr(lib, name)
    assert sorted(_lib.EXPORTED_SYMBOLS) == _declared_functions()


def test_library_identity_queries():
    from spconv_triton.pytorch._impl import _lib

    L = _lib.load_library()
    assert L.sp_arch() == b"gfx950"
    assert L.sp_version() == (0 << 16) | (1 << 8)
    header = (ROOT / "include" / "spconv_hip.h").read_text()
    m = re.search(r"#define SP_ABI_VERSION (\d+)", header)
    assert m and L.sp_abi_version() == int(m.group(1)) == _lib.ABI_VERSION


def _geom(mode, shape, out_shape, ks=3, st=1, pad=1, dil=1, batch=1):
    from spconv_triton.pytorch._impl import _lib

    nd = len(shape)
    return _lib.make_geom(mode, batch, shape, out_shape, [ks] * nd, [st] * nd, [pad] * nd,
                          [dil] * nd)


def test_key_width_rule_matches_reference():
    """int64 keys iff batch * volume >= 2^31 (reference pairs.py:166-171)."""
    from spconv_triton.pytorch._impl import _lib, pairs

    L = _lib.load_library()
    cases = [
        ([41, 1600, 1408], 4, False),       # 3.69e8
        ([2048, 2048, 128], 2, False),      # 1.07e9
        ([2048, 2048, 256], 2, True),       # 2.15e9
        ([512, 512, 512], 16, True),
        ([1290, 1290, 1290], 1, False),     # 2.147e9 - 1 > ... just below?
    ]
    for shape, batch, expect in cases:
        vol = batch * shape[0] * shape[1] * shape[2]
        exp = vol >= 2 ** 31
        g = _geom(_lib.SP_PAIR_SUBM, shape, shape, batch=batch)
        assert L.sp_geom_key64(ctypes.byref(g)) == int(exp)
        assert pairs.key_is_int64(batch, shape, shape, True) == exp
        if shape != [1290, 1290, 1290]:
            assert exp == expect


def test_workspace_queries_and_bad_geometry():
    from spconv_triton.pytorch._impl import _lib

    L = _lib.load_library()
    g = _geom(_lib.SP_PAIR_SUBM, [64, 64, 64], [64, 64, 64])
    assert L.sp_pairgen_workspace_size(ctypes.byref(g), 1000) >= 2048 * 8
    g2 = _geom(_lib.SP_PAIR_REGULAR, [64, 64, 64], [32, 32, 32], st=2)
    assert L.sp_pairgen_workspace_size(ctypes.byref(g2), 1000) > 0
    assert L.sp_mask_sort_workspace_size(200000, 1) > 0
    assert L.sp_conv_packed_bytes(64, 27, 64, _lib.SP_F16, 0) >= 27 * 64 * 64 * 2
    # even subm kernels are rejected by the geometry check (host-only path)
    bad = _geom(_lib.SP_PAIR_SUBM, [8, 8, 8], [8, 8, 8], ks=2)
    assert L.sp_geom_key64(ctypes.byref(bad)) == -1
    assert b"odd" in L.sp_last_error()
    # the ordered GEMM's kernel mode is checked before anything runs (M = 0)
    order = (ctypes.c_int32 * 1)(0)
    for thin, rc in ((0, 0), (2, 0), (3, _lib.SP_ERR_INVALID_ARG), (-1, _lib.SP_ERR_INVALID_ARG)):
        assert L.sp_conv_gemm_ordered(None, _lib.SP_F16, 0, None, 8, 27, 8, 0, 0, None, 0, order,
                                      None, 0, thin, None, 0, None, _lib.SP_F16, None) == rc
    assert b"thin_tiles" in L.sp_last_error()


def test_error_mapping():
    from spconv_triton.pytorch._impl import _lib

    with pytest.raises(ValueError):
        _lib.check(_lib.SP_ERR_INVALID_ARG, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.SP_ERR_UNSUPPORTED, "x")
    with pytest.raises(_lib.SpconvHipError):
        _lib.check(_lib.SP_ERR_HIP, "x")


def test_public_api_matches_reference():
    import spconv_triton
    import spconv_triton.pytorch as spconv

    api = json.loads((ROOT / "tests" / "golden" / "api.json").read_text())
    for name in api["pytorch"]:
        assert hasattr(spconv, name), name
    for name in api["ops"]:
        assert hasattr(spconv.ops, name), name
    for name in api["top"]:
        assert hasattr(spconv_triton, name), name
    for name in api["functional"]:
        assert hasattr(spconv.functional, name), name
    from spconv_triton.pytorch import hash as sp_hash
    from spconv_triton.pytorch import utils as sp_utils

    for name in api["hash"]:
        assert hasattr(sp_hash, name), name
    for name in api["pytorch_utils"]:
        assert hasattr(sp_utils, name), name
    for cls, args in api["ctors"].items():
        params = list(inspect.signature(getattr(spconv, cls).__init__).parameters)[1:]
        assert params == args, f"{cls}: {params} != {args}"


def test_gpu_ops_reject_cpu_tensors():
    """The product path never falls back to the CPU."""
    import torch

    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    idx = torch.zeros((4, 4), dtype=torch.int32)
    with pytest.raises(AssertionError):
        ops.get_indice_pairs_implicit_gemm(idx, 1, [8, 8, 8], ConvAlgo.MaskImplicitGemm,
                                           [3] * 3, [1] * 3, [1] * 3, [1] * 3, [0] * 3, True)
    with pytest.raises(AssertionError):
        ops.get_indice_pairs(idx, 1, [8, 8, 8], ConvAlgo.Native, [3] * 3, [1] * 3, [1] * 3,
                             [1] * 3, [0] * 3, True)


def test_module_construction_and_state_dict_layout(golden):
    """KRSC parameter layout and Kaiming bounds (no GPU)."""
    import math

    import torch

    import spconv_triton.pytorch as spconv

    m = spconv.SubMConv3d(64, 32, 3, indice_key="k")
    assert tuple(m.weight.shape) == (32, 3, 3, 3, 64)
    bound = math.sqrt(3.0) * math.sqrt(2.0 / 6.0) / math.sqrt(64 * 27)
    assert float(m.weight.abs().max()) <= bound + 1e-7
    assert m.algo == spconv.ConvAlgo.MaskImplicitGemm
    big = spconv.SubMConv3d(8, 8, 5)
    assert big.algo == spconv.ConvAlgo.Native
    assert spconv.SubMConv3d(8, 8, 5, large_kernel_fast_algo=True).algo == \
        spconv.ConvAlgo.MaskImplicitGemm
    case = golden("proto.pt", "init_subm3d")
    torch.manual_seed(case["seed"])
    layer = getattr(spconv, case["cls"])(**case["ctor"])
    for name, value in case["expect"].items():
        if isinstance(value, torch.Tensor) and hasattr(layer, name):
            assert torch.equal(getattr(layer, name).detach(), value), name
