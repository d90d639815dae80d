"""Small helpers re-exported by spconv's ``utils`` package."""

from contextlib import nullcontext

__all__ = ["nullcontext"]
