"""Identity module accepting and ignoring extra arguments (spconv.pytorch.identity)."""

from torch import nn


class Identity(nn.Module):
    def forward(self, input, *args, **kwargs):
        return input
