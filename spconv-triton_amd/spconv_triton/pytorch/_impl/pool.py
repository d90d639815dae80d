"""Sparse max/avg pooling host wrappers.

Host-side mirror of ``spconv_triton/pytorch/_impl/pool.py`` of the reference
(``maxpool_forward`` :260-284, ``maxpool_backward`` :287-330,
``avgpool_forward`` :333-367, ``avgpool_backward`` :370-397), running the
kernels of ``csrc/sp_pool.hip``.  Results are bit-identical to the reference:
pooling reductions do not depend on tiling (fp32 accumulator, fp64 for double).
"""

from __future__ import annotations

import torch

from . import _lib


def maxpool_forward(features: torch.Tensor, pair_fwd: torch.Tensor, n_out: int) -> torch.Tensor:
    _lib.require_gpu(features, pair_fwd)
    kv = pair_fwd.shape[0]
    x = features.contiguous()
    C = x.shape[1]
    out = torch.empty((n_out, C), dtype=x.dtype, device=x.device)
    if n_out == 0 or C == 0:
        return out
    pf = pair_fwd.contiguous()
    _lib.check(_lib.lib().sp_maxpool_fwd(_lib.ptr(x), _lib.dtype_code(x.dtype), x.shape[0], C,
                                         _lib.ptr(pf), kv, n_out, _lib.ptr(out),
                                         _lib.stream_of(x.device)), "sp_maxpool_fwd")
    return out


def maxpool_backward(features: torch.Tensor, out_features: torch.Tensor, grad_out: torch.Tensor,
                     pair_bwd: torch.Tensor) -> torch.Tensor:
    _lib.require_gpu(features, out_features, grad_out, pair_bwd)
    kv = pair_bwd.shape[0]
    x = features.contiguous()
    out = out_features.contiguous()
    g = grad_out.contiguous().to(x.dtype)
    n_in, C = x.shape
    din = torch.empty_like(x)
    if n_in == 0 or C == 0:
        return din
    pb = pair_bwd.contiguous()
    _lib.check(_lib.lib().sp_maxpool_bwd(_lib.ptr(x), _lib.ptr(out), _lib.ptr(g),
                                         _lib.dtype_code(x.dtype), n_in, C, _lib.ptr(pb), kv,
                                         out.shape[0], _lib.ptr(din), _lib.stream_of(x.device)),
               "sp_maxpool_bwd")
    return din


def avgpool_forward(features: torch.Tensor, pair_fwd: torch.Tensor, n_out: int,
                    calc_count: bool = True):
    _lib.require_gpu(features, pair_fwd)
    kv = pair_fwd.shape[0]
    x = features.contiguous()
    C = x.shape[1]
    out = torch.empty((n_out, C), dtype=x.dtype, device=x.device)
    count = torch.zeros((n_out,), dtype=torch.int32, device=x.device)
    if n_out == 0 or C == 0:
        return out, count
    pf = pair_fwd.contiguous()
    _lib.check(_lib.lib().sp_avgpool_fwd(_lib.ptr(x), _lib.dtype_code(x.dtype), x.shape[0], C,
                                         _lib.ptr(pf), kv, n_out, _lib.ptr(out), _lib.ptr(count),
                                         _lib.stream_of(x.device)), "sp_avgpool_fwd")
    return out, count


def avgpool_backward(grad_out: torch.Tensor, pair_bwd: torch.Tensor,
                     count: torch.Tensor) -> torch.Tensor:
    _lib.require_gpu(grad_out, pair_bwd, count)
    kv = pair_bwd.shape[0]
    g = grad_out.contiguous()
    n_in = pair_bwd.shape[1]
    C = g.shape[1]
    din = torch.empty((n_in, C), dtype=g.dtype, device=g.device)
    if n_in == 0 or C == 0:
        return din
    pb = pair_bwd.contiguous()
    cnt = count.contiguous().to(torch.int32)
    _lib.check(_lib.lib().sp_avgpool_bwd(_lib.ptr(g), _lib.ptr(cnt), _lib.dtype_code(g.dtype),
                                         g.shape[0], C, _lib.ptr(pb), kv, n_in, _lib.ptr(din),
                                         _lib.stream_of(g.device)), "sp_avgpool_bwd")
    return din
