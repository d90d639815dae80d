# SPDX-FileCopyrightText: Copyright contributors to the spconv-Triton project
# SPDX-FileCopyrightText: Derived from spconv, Copyright 2021 Yan Yan and contributors
# SPDX-License-Identifier: Apache-2.0
# The public names, signatures and error messages in this file follow spconv-Triton's
# API (Apache-2.0); the implementation is this package's own.
"""Sparse convolution modules (API and behaviour of spconv.pytorch.conv).

Mirror of reference ``spconv_triton/pytorch/conv.py``:

* algorithm choice: MaskImplicitGemm for kv <= 32 (128 with
  ``large_kernel_fast_algo``), Native above (:95-103);
* conv1x1 (kv == 1, stride 1) is a plain ``X @ weight.view(Cin, Cout)`` -- a
  raw reinterpretation of the KRSC storage, as upstream (:194-206);
* ``indice_key`` rulebook reuse with the reference's validation (:211-245,
  :515-567) and the pair_fwd/pair_bwd swap for inverse convs (:347-365);
* training adds the bias after the kernel, eval fuses it and returns the
  weight dtype (:141-142, :453-481);
* KRSC weight ``[Cout, *ksize, Cin]``, Kaiming-uniform init with a KRSC fan
  (:737-757), and the load hook with upstream's double permute (:655-698).
"""

from __future__ import annotations

import math
import time as _time

import numpy as np
import torch
from torch.nn import init
from torch.nn.init import calculate_gain
from torch.nn.parameter import Parameter

from spconv_triton import SPCONV_VERSION_NUMBERS  # noqa: F401
from spconv_triton.compat import Activation, tv
from spconv_triton.constants import SAVED_WEIGHT_LAYOUT, SPCONV_DEBUG_WEIGHT
from spconv_triton.core import ConvAlgo
from spconv_triton.pytorch import functional as Fsp
from spconv_triton.pytorch import ops
from spconv_triton.pytorch.core import (
    ImplicitGemmIndiceData,
    IndiceData,
    SparseConvTensor,
    expand_nd,
    register_implicit_gemm_indice_data,
)
from spconv_triton.pytorch.modules import SparseModule
from spconv_triton.utils import nullcontext  # noqa: F401

FILTER_HWIO = False
CPU_ONLY_BUILD = False

_MAX_NUM_VOXELS_DURING_TRAINING = "max_num_voxels_during_training"
_NO_ACT = tv.gemm.Activation.None_


def _default_algo(kv: int, large_kernel_fast_algo: bool) -> ConvAlgo:
    limit = 128 if large_kernel_fast_algo else 32
    return ConvAlgo.MaskImplicitGemm if kv <= limit else ConvAlgo.Native


class SparseConvolutionBase:
    def __init__(self, ndim: int, in_channels: int, out_channels: int, kernel_size=3, stride=1,
                 padding=0, dilation=1, groups: int = 1, bias: bool = True, subm: bool = False,
                 output_padding=0, transposed: bool = False, inverse: bool = False,
                 indice_key: str | None = None, algo: ConvAlgo | None = None,
                 fp32_accum: bool | None = None, record_voxel_count: bool = False,
                 act_type: Activation = _NO_ACT, act_alpha: float = 0, act_beta: float = 0,
                 large_kernel_fast_algo: bool = False):
        if groups != 1:
            raise AssertionError("don't support groups for now")
        self.ndim = ndim
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = expand_nd(ndim, kernel_size)
        self.stride = expand_nd(ndim, stride)
        self.dilation = expand_nd(ndim, dilation)
        self.padding = expand_nd(ndim, padding)
        self.output_padding = expand_nd(ndim, output_padding)
        kv = int(np.prod(self.kernel_size))
        self.conv1x1 = kv == 1 and (subm or int(np.prod(self.stride)) == 1)
        if self.conv1x1 and not subm and self.padding != [0] * ndim:
            raise AssertionError("padding must be zero for 1x1 conv (k=1,s=1)")
        self.transposed = transposed
        self.inverse = inverse
        self.groups = groups
        self.subm = subm
        self.indice_key = indice_key
        self.record_voxel_count = record_voxel_count
        self.algo = algo if algo is not None else _default_algo(kv, large_kernel_fast_algo)
        self.fp32_accum = fp32_accum
        self.weight_shape = [out_channels, *self.kernel_size, in_channels]
        self.act_type = act_type
        self.act_alpha = act_alpha
        self.act_beta = act_beta
        if self.conv1x1 and act_type != _NO_ACT:
            raise AssertionError("conv1x1 don't support fused act")

    def is_inverseable(self):
        return self.indice_key is not None and not self.subm

    # ------------------------------------------------------------------
    def _out_spatial_shape(self, spatial_shape):
        if self.subm:
            return spatial_shape
        if self.transposed:
            return ops.get_deconv_output_size(spatial_shape, self.kernel_size, self.stride,
                                              self.padding, self.dilation, self.output_padding)
        return ops.get_conv_output_size(spatial_shape, self.kernel_size, self.stride,
                                        self.padding, self.dilation)

    def _bench_entry(self, x: SparseConvTensor, name):
        if name is None:
            raise ValueError("you need to assign name to spmodules before benchmark "
                             "(spconv.utils.bench.assign_name_to_spmod)")
        if name not in x.benchmark_record:
            x.benchmark_record[name] = {
                "type": "SparseConvolution", "indice_gen_time": [], "time": [],
                "num_points": [], "num_out_points": [],
                "params": {"kernel_size": self.kernel_size, "stride": self.stride,
                           "padding": self.padding, "dilation": self.dilation,
                           "output_padding": self.output_padding, "subm": self.subm,
                           "transposed": self.transposed, "input_channels": self.in_channels,
                           "out_channels": self.out_channels},
            }

    def _conv_forward(self, training: bool, x: SparseConvTensor, weight: torch.Tensor,
                      bias: torch.Tensor | None, add_input: SparseConvTensor | None = None,
                      channel_scale: torch.Tensor | None = None,
                      output_scale: float | None = None, name: str | None = None,
                      act_type: Activation = _NO_ACT, act_alpha: float = 0,
                      act_beta: float = 0):
        if x.is_quantized and weight.is_quantized:
            raise NotImplementedError("int8 is not supported by spconv_triton")
        if x.features.shape[1] != self.in_channels:
            raise AssertionError("channel size mismatch")
        if training and self.act_type != _NO_ACT:
            raise AssertionError("act don't support backward, only used in inference")
        features = x.features
        spatial_shape = x.spatial_shape
        out_spatial_shape = self._out_spatial_shape(spatial_shape)
        out_tensor = x.shadow_copy()
        if x.benchmark:
            self._bench_entry(x, name)

        if self.conv1x1:
            out = torch.mm(x.features, weight.view(self.in_channels, self.out_channels))
            if bias is not None:
                out += bias
            out_tensor = out_tensor.replace_feature(out)
            out_tensor.spatial_shape = out_spatial_shape
            return out_tensor

        indice_dict = x.indice_dict.copy()
        features = features.contiguous()
        datas = x.find_indice_pair(self.indice_key)
        if datas is not None and self.algo != datas.algo:
            raise AssertionError("due to limitation of pytorch, you must provide same algo to "
                                 "layers share same indice key.")
        bias_infer = None if training else bias
        bench_t = None

        def timed_pairgen(fn):
            if not x.benchmark:
                return fn()
            torch.cuda.synchronize()
            t0 = _time.time()
            res = fn()
            torch.cuda.synchronize()
            out_tensor.benchmark_record[name]["indice_gen_time"].append(_time.time() - t0)
            return res

        if self.algo == ConvAlgo.Native:
            if datas is not None and not isinstance(datas, IndiceData):
                raise AssertionError
            if self.inverse:
                self._require_inverse_source(datas)
                outids = datas.indices
                pairs, pair_num = datas.indice_pairs, datas.indice_pair_num
                out_spatial_shape = datas.spatial_shape
                self._check_inverse_reuse_valid(x, spatial_shape, datas)
            elif datas is not None:
                if not self.subm:
                    raise AssertionError("only support reuse subm indices")
                outids = datas.out_indices
                pairs, pair_num = datas.indice_pairs, datas.indice_pair_num
                self._check_subm_reuse_valid(x, spatial_shape, datas)
            else:
                outids, pairs, pair_num = timed_pairgen(lambda: ops.get_indice_pairs(
                    x.indices, x.batch_size, spatial_shape, self.algo, self.kernel_size,
                    self.stride, self.padding, self.dilation, self.output_padding, self.subm,
                    self.transposed))
                if self.indice_key is not None:
                    if self.indice_key in indice_dict:
                        raise AssertionError(f"your indice key {self.indice_key} already "
                                             f"exists in this sparse tensor.")
                    indice_dict[self.indice_key] = IndiceData(
                        outids, x.indices, pairs, pair_num, spatial_shape, out_spatial_shape,
                        is_subm=self.subm, algo=self.algo, ksize=self.kernel_size,
                        stride=self.stride, padding=self.padding, dilation=self.dilation)
            if x.benchmark:
                torch.cuda.synchronize()
                bench_t = _time.time()
            if pairs.device != features.device:
                pairs = pairs.to(features.device)
            if self.subm:
                fn = Fsp.indice_subm_conv
            elif self.inverse:
                fn = Fsp.indice_inverse_conv
            else:
                fn = Fsp.indice_conv
            # upstream passes act_type in the act_alpha slot for regular convs;
            # it is inert because act_type stays None_ on that path
            alpha = act_type if fn is Fsp.indice_conv else act_alpha
            out_features = fn(features, weight, pairs, pair_num, outids.shape[0], self.algo,
                              x._timer, bias_infer, alpha, act_beta, act_type)
        else:
            if datas is not None and not isinstance(datas, ImplicitGemmIndiceData):
                raise AssertionError
            if self.inverse:
                self._require_inverse_source(datas)
                outids = datas.indices
                pair_fwd, pair_bwd = datas.pair_bwd, datas.pair_fwd
                masks = datas.masks
                out_spatial_shape = datas.spatial_shape
                self._check_inverse_reuse_valid(x, spatial_shape, datas)
            elif datas is not None:
                outids = datas.out_indices
                pair_fwd, pair_bwd = datas.pair_fwd, datas.pair_bwd
                masks = datas.masks
                if not self.subm:
                    raise AssertionError("only support reuse subm indices")
                self._check_subm_reuse_valid(x, spatial_shape, datas)
            else:
                # the mask sorts are deferred: the gather-GEMM does not read them
                res, deferred = timed_pairgen(lambda: ops.implicit_gemm_rulebook(
                    x.indices, x.batch_size, spatial_shape, self.algo, ksize=self.kernel_size,
                    stride=self.stride, padding=self.padding, dilation=self.dilation,
                    out_padding=self.output_padding, subm=self.subm, transpose=self.transposed,
                    is_train=(not self.subm) or training))
                outids, pair_fwd, pair_bwd, masks = res[0], res[2], res[3], res[8]
                if self.indice_key is not None:
                    register_implicit_gemm_indice_data(
                        indice_dict, self.indice_key, res, x.indices, is_subm=self.subm,
                        spatial_shape=spatial_shape, out_spatial_shape=out_spatial_shape,
                        algo=self.algo, ksize=self.kernel_size, stride=self.stride,
                        dilation=self.dilation, padding=self.padding, deferred_masks=deferred)
            # the kernels skip offsets without pairs themselves; the sorted
            # mask splits would not change the result and are not passed
            pm_fwd = pm_bwd = ma_fwd = ma_bwd = []
            if x.benchmark:
                torch.cuda.synchronize()
                bench_t = _time.time()
            n_act = outids.shape[0]
            if training:
                out_features = Fsp.implicit_gemm(features, weight, pair_fwd, pair_bwd, pm_fwd,
                                                 pm_bwd, ma_fwd, ma_bwd, n_act, masks, training,
                                                 self.subm, x._timer, self.fp32_accum,
                                                 bias_infer, act_alpha, act_beta, act_type)
            else:
                out_dtype = weight.dtype if output_scale is None else None
                out_features, _, _ = ops.implicit_gemm(
                    features, weight, pair_fwd, pm_fwd, ma_fwd, n_act, masks, training,
                    self.subm, x._timer, self.fp32_accum, bias_infer, act_alpha, act_beta,
                    act_type, 1.0 if output_scale is None else output_scale, channel_scale,
                    output_add=add_input.features if add_input is not None else None,
                    output_add_scale=0.0, output_dtype=out_dtype)

        if training and bias is not None:
            out_features += bias
        if x.benchmark:
            torch.cuda.synchronize()
            rec = out_tensor.benchmark_record[name]
            rec["time"].append(_time.time() - bench_t)
            rec["num_points"].append(features.shape[0])
            rec["num_out_points"].append(out_features.shape[0])
        if (not self.subm and not self.inverse and self.record_voxel_count
                and hasattr(self, _MAX_NUM_VOXELS_DURING_TRAINING)):
            ops.maximum_value_int_(getattr(self, _MAX_NUM_VOXELS_DURING_TRAINING),
                                   outids.shape[0])
        out_tensor = out_tensor.replace_feature(out_features)
        out_tensor.indices = outids
        out_tensor.indice_dict = indice_dict
        out_tensor.spatial_shape = out_spatial_shape
        if add_input is not None:
            out_tensor = out_tensor.replace_feature(ops._apply_act_inplace(
                out_tensor.features + add_input.features, self.act_type, self.act_alpha,
                self.act_beta))
        return out_tensor

    def _require_inverse_source(self, datas):
        if datas is None:
            raise AssertionError
        if self.indice_key is None:
            raise AssertionError
        if datas.is_subm is not False:
            raise AssertionError("inverse conv can only be used with standard conv and pool ops.")

    def _check_subm_reuse_valid(self, inp: SparseConvTensor, spatial_shape, datas):
        if not datas.is_subm:
            raise AssertionError("only support reuse subm indices")
        if self.kernel_size != datas.ksize:
            raise ValueError(f"subm with same indice_key must have same kernel size, expect "
                             f"{datas.ksize}, this layer {self.kernel_size}")
        if self.dilation != datas.dilation:
            raise ValueError(f"subm with same indice_key must have same dilation, expect "
                             f"{datas.dilation}, this layer {self.dilation}")
        if inp.spatial_shape != datas.spatial_shape:
            raise ValueError(f"subm with same indice_key must have same spatial structure, "
                             f"expect {datas.spatial_shape}, input {spatial_shape}")
        if inp.indices.shape[0] != datas.indices.shape[0]:
            raise ValueError(f"subm with same indice_key must have same num of indices, expect "
                             f"{datas.indices.shape[0]}, input {inp.indices.shape[0]}")

    def _check_inverse_reuse_valid(self, inp: SparseConvTensor, spatial_shape, datas):
        if self.kernel_size != datas.ksize:
            raise ValueError(f"Inverse with same indice_key must have same kernel size, expect "
                             f"{datas.ksize}, this layer {self.kernel_size}, please check "
                             "Inverse Convolution in docs/USAGE.md.")
        if inp.spatial_shape != datas.out_spatial_shape:
            raise ValueError(f"Inverse with same indice_key must have same spatial structure "
                             f"(spatial shape), expect {datas.spatial_shape}, input "
                             f"{spatial_shape}, please check Inverse Convolution in "
                             "docs/USAGE.md.")
        if inp.indices.shape[0] != datas.out_indices.shape[0]:
            raise ValueError(f"Inverse with same indice_key must have same num of indices, "
                             f"expect {datas.indices.shape[0]}, input {inp.indices.shape[0]}, "
                             "please check Inverse Convolution in .")


class SparseConvolution(SparseConvolutionBase, SparseModule):
    __constants__ = ["stride", "padding", "dilation", "groups", "bias", "subm", "inverse",
                     "transposed", "output_padding"]

    def __init__(self, ndim: int, in_channels: int, out_channels: int, kernel_size=3, stride=1,
                 padding=0, dilation=1, groups: int = 1, bias: bool = True, subm: bool = False,
                 output_padding=0, transposed: bool = False, inverse: bool = False,
                 indice_key: str | None = None, algo: ConvAlgo | None = None,
                 fp32_accum: bool | None = None, record_voxel_count: bool = False,
                 act_type: Activation = _NO_ACT, act_alpha: float = 0, act_beta: float = 0,
                 large_kernel_fast_algo: bool = False, name=None, device=None, dtype=None):
        SparseConvolutionBase.__init__(
            self, ndim, in_channels, out_channels, kernel_size, stride, padding, dilation,
            groups, bias=False, subm=subm, output_padding=output_padding, transposed=transposed,
            inverse=inverse, indice_key=indice_key, algo=algo, fp32_accum=fp32_accum,
            record_voxel_count=record_voxel_count, act_type=act_type, act_alpha=act_alpha,
            act_beta=act_beta, large_kernel_fast_algo=large_kernel_fast_algo)
        SparseModule.__init__(self, name=name)
        factory = {"device": device, "dtype": dtype}
        if record_voxel_count and not self.subm and not self.inverse:
            self.register_buffer(_MAX_NUM_VOXELS_DURING_TRAINING,
                                 torch.zeros(1, dtype=torch.int32, device=device))
        self.weight = Parameter(torch.zeros(*self.weight_shape, **factory))
        if bias:
            self.bias = Parameter(torch.zeros(out_channels, **factory))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()
        self._register_load_state_dict_pre_hook(self._load_weight_different_layout)

    def get_max_num_voxels(self) -> torch.Tensor | None:
        return getattr(self, _MAX_NUM_VOXELS_DURING_TRAINING, None)

    def _load_weight_different_layout(self, state_dict, prefix, local_metadata, strict,
                                      missing_keys, unexpected_keys, error_msgs):
        key = prefix + _MAX_NUM_VOXELS_DURING_TRAINING
        if (self.record_voxel_count and not self.subm and not self.inverse
                and key not in state_dict):
            state_dict[key] = torch.zeros(1, dtype=torch.int32)
        if not SAVED_WEIGHT_LAYOUT:
            return
        wkey = prefix + "weight"
        if wkey not in state_dict:
            raise AssertionError
        nd = self.ndim
        if SAVED_WEIGHT_LAYOUT == "RSKC":
            perm = (nd, *range(nd), nd + 1)
        elif SAVED_WEIGHT_LAYOUT == "RSCK":
            perm = (nd + 1, *range(nd), nd)
        else:
            return
        # upstream spconv 2.3.8 applies the permute twice, so a non-KRSC
        # checkpoint always fails to load on a shape mismatch; kept as is.
        for _ in range(2):
            state_dict[wkey] = state_dict[wkey].permute(*perm).contiguous()

    def extra_repr(self):
        s = "{in_channels}, {out_channels}, kernel_size={kernel_size}, stride={stride}"
        if self.padding != (0,) * len(self.padding):
            s += ", padding={padding}"
        if self.dilation != (1,) * len(self.dilation):
            s += ", dilation={dilation}"
        if self.output_padding != (0,) * len(self.output_padding):
            s += ", output_padding={output_padding}"
        if self.groups != 1:
            s += ", groups={groups}"
        if self.bias is None:
            s += ", bias=False"
        if self.algo is not None:
            s += f", algo={self.algo}"
        if self.act_type != _NO_ACT:
            s += f", act={self.act_type}"
        return s.format(**self.__dict__)

    def _calculate_fan_in_and_fan_out(self):
        receptive = int(np.prod(self.kernel_size))
        return self.in_channels * receptive, self.out_channels * receptive

    def _calculate_correct_fan(self, mode):
        mode = mode.lower()
        if mode not in ("fan_in", "fan_out"):
            raise ValueError(f"Mode {mode} not supported, please use one of "
                             f"['fan_in', 'fan_out']")
        fan_in, fan_out = self._calculate_fan_in_and_fan_out()
        return fan_in if mode == "fan_in" else fan_out

    def _custom_kaiming_uniform_(self, tensor, a=0, mode="fan_in", nonlinearity="leaky_relu"):
        """kaiming_uniform_ with the fan computed for the KRSC layout."""
        bound = math.sqrt(3.0) * calculate_gain(nonlinearity, a) / math.sqrt(
            self._calculate_correct_fan(mode))
        with torch.no_grad():
            return tensor.uniform_(-bound, bound)

    def reset_parameters(self):
        self._custom_kaiming_uniform_(self.weight,
                                      a=math.sqrt(0.005 if SPCONV_DEBUG_WEIGHT else 5))
        if self.bias is not None:
            fan_in, _ = self._calculate_fan_in_and_fan_out()
            bound = 1 / math.sqrt(fan_in)
            init.uniform_(self.bias, -bound, bound)

    @torch.compiler.disable
    def forward(self, x: SparseConvTensor, add_input: SparseConvTensor | None = None):
        return self._conv_forward(self.training, x, self.weight, self.bias, add_input,
                                  name=self.name, act_type=self.act_type,
                                  act_alpha=self.act_alpha, act_beta=self.act_beta)


# ---------------------------------------------------------------------------
# leaf classes: constructor signatures of spconv 2.3.8
# ---------------------------------------------------------------------------

def _make_regular(ndim: int, transposed: bool):
    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1,
                 groups=1, bias=True, indice_key=None, algo: ConvAlgo | None = None,
                 fp32_accum: bool | None = None, record_voxel_count: bool = False,
                 large_kernel_fast_algo: bool = False, name=None):
        SparseConvolution.__init__(self, ndim, in_channels, out_channels, kernel_size, stride,
                                   padding, dilation, groups, bias, transposed=transposed,
                                   indice_key=indice_key, algo=algo, fp32_accum=fp32_accum,
                                   record_voxel_count=record_voxel_count,
                                   large_kernel_fast_algo=large_kernel_fast_algo, name=name)
    return __init__


def _make_subm(ndim: int):
    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1,
                 groups=1, bias=True, indice_key=None, algo: ConvAlgo | None = None,
                 fp32_accum: bool | None = None, large_kernel_fast_algo: bool = False,
                 name=None):
        SparseConvolution.__init__(self, ndim, in_channels, out_channels, kernel_size, stride,
                                   padding, dilation, groups, bias, True, indice_key=indice_key,
                                   algo=algo, fp32_accum=fp32_accum,
                                   large_kernel_fast_algo=large_kernel_fast_algo, name=name)
    return __init__


def _make_inverse(ndim: int):
    def __init__(self, in_channels, out_channels, kernel_size, indice_key, bias=True,
                 algo: ConvAlgo | None = None, fp32_accum: bool | None = None,
                 large_kernel_fast_algo: bool = False, name=None):
        SparseConvolution.__init__(self, ndim, in_channels, out_channels, kernel_size, bias=bias,
                                   inverse=True, indice_key=indice_key, algo=algo,
                                   fp32_accum=fp32_accum,
                                   large_kernel_fast_algo=large_kernel_fast_algo, name=name)
    return __init__


class SparseConv1d(SparseConvolution):
    __init__ = _make_regular(1, False)


class SparseConv2d(SparseConvolution):
    __init__ = _make_regular(2, False)


class SparseConv3d(SparseConvolution):
    __init__ = _make_regular(3, False)


class SparseConv4d(SparseConvolution):
    __init__ = _make_regular(4, False)


class SparseConvTranspose1d(SparseConvolution):
    __init__ = _make_regular(1, True)


class SparseConvTranspose2d(SparseConvolution):
    __init__ = _make_regular(2, True)


class SparseConvTranspose3d(SparseConvolution):
    __init__ = _make_regular(3, True)


class SparseConvTranspose4d(SparseConvolution):
    __init__ = _make_regular(4, True)


class SparseInverseConv1d(SparseConvolution):
    __init__ = _make_inverse(1)


class SparseInverseConv2d(SparseConvolution):
    __init__ = _make_inverse(2)


class SparseInverseConv3d(SparseConvolution):
    __init__ = _make_inverse(3)


class SparseInverseConv4d(SparseConvolution):
    __init__ = _make_inverse(4)


class SubMConv1d(SparseConvolution):
    __init__ = _make_subm(1)


class SubMConv2d(SparseConvolution):
    __init__ = _make_subm(2)


class SubMConv3d(SparseConvolution):
    __init__ = _make_subm(3)


class SubMConv4d(SparseConvolution):
    __init__ = _make_subm(4)
