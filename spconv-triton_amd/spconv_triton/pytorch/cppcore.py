"""Stream helper of spconv.pytorch.cppcore (no cumm/tensorview here)."""

import torch


def get_current_stream() -> int:
    if torch.cuda.is_available():
        return torch.cuda.current_stream().cuda_stream
    return 0


def torch_tensor_to_tv(*args, **kwargs):
    raise NotImplementedError("spconv_triton has no cumm/tensorview backend; "
                              "use plain torch tensors.")
