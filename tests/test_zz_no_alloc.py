"""sp_conv_fwd_noalloc: the forward with its relaid weights in the library's
per-GPU scratch array instead of a caller workspace.  Called through the C
ABI and compared bit for bit with sp_conv_fwd (same kernels, same summation
order) on two calls in a row, the second on a smaller input, in each compute
dtype; sizes above SP_NOALLOC_SCRATCH_BYTES are rejected with
SP_ERR_UNSUPPORTED before any work is enqueued; and the call allocates
nothing (free device memory unchanged across calls, replays of a captured
graph equal to the workspace forward).
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


def test_noalloc_allocates_nothing():
    """The entry point's contract: after the first call on the device (which
    looks up the scratch array's address), calls of other sizes leave the
    device's free memory unchanged, and the call can be captured into a HIP
    graph whose replays -- with eager work and synchronisations between them
    -- equal the workspace forward each time."""
    from spconv_triton.pytorch._impl import _lib

    L = _lib.lib()
    dt = _lib.dtype_code(torch.float16)
    cases = []
    for i, (n, grid, C, K) in enumerate(((9000, 36, 64, 64), (2500, 20, 16, 32))):
        pf, _, _ = _rulebook(n, grid, seed=30 + i)
        torch.manual_seed(20 + i)
        x = torch.randn(n, C, device=DEV).half()
        w = (torch.randn(K, 27, C, device=DEV) / np.sqrt(27 * C)).half()
        b = torch.randn(K, device=DEV).half()
        out = torch.empty((n, K), dtype=torch.float16, device=DEV)
        cases.append((x, w, b, pf, out))

    def call(x, w, b, pf, out):
        K, kv, C = w.shape
        _lib.check(L.sp_conv_fwd_noalloc(_lib.ptr(x), dt, x.shape[0], C, _lib.ptr(w), dt, K, kv,
                                         _lib.ptr(pf), pf.shape[1], _lib.ptr(b), None, None,
                                         _lib.ptr(out), dt, _lib.stream_of(x.device)),
                   "sp_conv_fwd_noalloc")

    call(*cases[0])  # warm-up: scratch address lookup
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(0)[0]
    for c in (cases[1], cases[0], cases[1]):
        call(*c)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(0)[0] == free0, "the no-allocation forward allocated memory"

    x, w, b, pf, out = cases[1]
    ref, _ = _both(x, w, b, pf, False, None, None, torch.float16)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(x, w, b, pf, out)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        out.fill_(float("nan"))
        call(*cases[0])  # eager use of the shared scratch between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"graph replay {rep} differs from the workspace forward"
