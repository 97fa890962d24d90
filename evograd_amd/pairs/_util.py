"""Argument checks shared by the pair modules."""

from __future__ import annotations

import torch

from evograd_amd import _lib


def as_contiguous(name: str, t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def check_same(name: str, ref: torch.Tensor, *others: torch.Tensor) -> None:
    for o in others:
        if o.dtype != ref.dtype:
            raise TypeError(f"{name}: dtype mismatch {ref.dtype} vs {o.dtype}")


def workspace(nbytes: int, device) -> torch.Tensor:
    """Scratch bytes from torch's caching allocator (the library never allocates)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


tag = _lib.dtype_tag
