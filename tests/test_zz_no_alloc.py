"""sp_conv_fwd_noalloc: the forward with its relaid weights in the library's
per-GPU scratch array instead of a caller workspace.  Called through the C
ABI and compared bit for bit with sp_conv_fwd (same kernels, same summation
order) on two calls in a row, the second on a smaller input, in each compute
dtype; sizes above SP_NOALLOC_SCRATCH_BYTES are rejected with
SP_ERR_UNSUPPORTED before any work is enqueued.
"""

import re
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ROOT = Path(__file__).resolve().parents[1]


def _scratch_bytes():
    text = (ROOT / "include" / "spconv_hip.h").read_text()
    m = re.search(r"#define SP_NOALLOC_SCRATCH_BYTES \((\d+) \* (\d+) \* (\d+)\)", text)
    return int(m.group(1)) * int(m.group(2)) * int(m.group(3))


def _rulebook(n, grid, seed):
    from spconv_triton.core import ConvAlgo
    from spconv_triton.pytorch import ops

    rng = np.random.default_rng(seed)
    lin = rng.choice(grid ** 3, size=n, replace=False)
    c = np.stack(np.unravel_index(lin, [grid] * 3), 1)
    idx = np.concatenate([np.zeros((n, 1)), c], 1).astype(np.int32)
    res = ops.get_indice_pairs_implicit_gemm(torch.from_numpy(idx).to(DEV), 1, [grid] * 3,
                                             ConvAlgo.MaskImplicitGemm, [3] * 3, [1] * 3,
                                             [1] * 3, [1] * 3, [0] * 3, True, is_train=False)
    return res[2], res[4][0][:, 0].contiguous(), res[6][0]


def _both(x, w, b, pf, masked, pm, ar, out_dtype):
    from spconv_triton.pytorch._impl import _lib

    L = _lib.lib()
    K, kv, C = w.shape
    n_out = pf.shape[1]
    dt, wdt, odt = (_lib.dtype_code(t) for t in (x.dtype, w.dtype, out_dtype))
    s = _lib.stream_of(x.device)
    ref = torch.empty((n_out, K), dtype=out_dtype, device=DEV)
    ws = torch.empty(L.sp_conv_workspace_size(K, kv, C, dt), dtype=torch.uint8, device=DEV)
    pmp, arp = (_lib.ptr(pm), _lib.ptr(ar)) if masked else (None, None)
    _lib.check(L.sp_conv_fwd(_lib.ptr(x), dt, x.shape[0], C, _lib.ptr(w), wdt, K, kv,
                             _lib.ptr(pf), n_out, _lib.ptr(b), pmp, arp, _lib.ptr(ref), odt,
                             _lib.ptr(ws), ws.numel(), s), "sp_conv_fwd")
    out = torch.full((n_out, K), float("nan"), dtype=out_dtype, device=DEV)
    _lib.check(L.sp_conv_fwd_noalloc(_lib.ptr(x), dt, x.shape[0], C, _lib.ptr(w), wdt, K, kv,
                                     _lib.ptr(pf), n_out, _lib.ptr(b), pmp, arp, _lib.ptr(out),
                                     odt, s), "sp_conv_fwd_noalloc")
    return ref, out


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_noalloc_forward_equals_workspace_forward(dtype):
    calls = [  # (voxels, grid, C, K, masked): the second call is smaller
        (12000, 40, 64, 96, False),
        (3000, 24, 32, 48, True),
    ]
    for i, (n, grid, C, K, masked) in enumerate(calls):
        pf, pm, ar = _rulebook(n, grid, seed=10 + i)
        torch.manual_seed(i)
        x = torch.randn(n, C, device=DEV).to(dtype)
        w = (torch.randn(K, 27, C, device=DEV) / np.sqrt(27 * C)).to(dtype)
        b = torch.randn(K, device=DEV).to(dtype)
        ref, out = _both(x, w, b, pf, masked, pm, ar, dtype)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"call {i}: noalloc forward differs"
        # without bias, fp32 output
        ref2, out2 = _both(x, w, None, pf, masked, pm, ar, torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(out2, ref2), f"call {i}: noalloc forward (no bias, f32 out) differs"


def test_noalloc_rejects_weights_beyond_scratch():
    from spconv_triton.pytorch._impl import _lib

    L = _lib.lib()
    limit = _scratch_bytes()
    f32 = _lib.dtype_code(torch.float32)
    K, kv, C = 512, 125, 256  # 64 MB of relaid fp32 weights
    assert L.sp_conv_workspace_size(K, kv, C, f32) > limit
    dummy = torch.zeros(16, dtype=torch.int32, device=DEV)
    p = _lib.ptr(dummy)
    rc = L.sp_conv_fwd_noalloc(p, f32, 1, C, p, f32, K, kv, p, 1, None, None, None, p, f32,
                               _lib.stream_of(dummy.device))
    assert rc == _lib.SP_ERR_UNSUPPORTED
    assert b"scratch" in L.sp_last_error()
