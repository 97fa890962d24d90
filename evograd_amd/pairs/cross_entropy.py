"""Hard-label mean cross entropy pair on gfx950.

Replaces the eager pair of src/evograd/ops/level1/cross_entropy/forward_ref.py:6-12
(``F.cross_entropy(logits.float(), target, reduction="mean", ignore_index=-100)``
cast to the logits dtype) with the backward rule declared at
cross_entropy/__init__.py:91-94: ``dlogits = dloss * (softmax(logits) -
onehot(target)) / n_valid``, zero on ignored rows; ``target`` receives no gradient.

Saved state: ``(logits, target, stats)``, where the inputs are kept by reference and
``stats`` is ``rows + 1`` fp32 values: the logsumexp of every row, then the count of
non-ignored rows. The backward never re-reduces a row: one read of the logits and
one write of dlogits.
"""

from __future__ import annotations

if not __package__:
    # Loaded from this file's path as a top-level candidate module (evograd's verify
    # and bench commands load a program that way): put the package root on sys.path.
    import pathlib as _pathlib
    import sys as _sys

    _ROOT = str(_pathlib.Path(__file__).resolve().parents[2])
    if _ROOT not in _sys.path:
        _sys.path.insert(0, _ROOT)

import torch

from evograd_amd import _lib
from evograd_amd.pairs._util import as_contiguous, tag, workspace

IGNORE_INDEX = -100


def _check(logits: torch.Tensor, target: torch.Tensor) -> None:
    _lib.require_gpu("cross_entropy", logits, target)
    if logits.dim() != 2:
        raise ValueError(f"cross_entropy: logits must be [rows, cols], got {tuple(logits.shape)}")
    if target.dim() != 1 or target.shape[0] != logits.shape[0]:
        raise ValueError(
            f"cross_entropy: target must be [rows]={logits.shape[0]}, got {tuple(target.shape)}"
        )
    if target.dtype != torch.int64:
        raise TypeError(f"cross_entropy: target must be int64, got {target.dtype}")


def cross_entropy_forward_with_saved(logits: torch.Tensor, target: torch.Tensor):
    _check(logits, target)
    logits = as_contiguous("logits", logits)
    target = as_contiguous("target", target)
    rows, cols = logits.shape
    loss = torch.empty((), dtype=logits.dtype, device=logits.device)
    stats = torch.empty(rows + 1, dtype=torch.float32, device=logits.device)
    ws = workspace(_lib.query("eg_cross_entropy_workspace_bytes", rows), logits.device)
    base = stats.data_ptr()
    _lib.call("eg_cross_entropy_fwd", _lib.ptr(logits), _lib.ptr(target), _lib.ptr(loss), base,
              base + 4 * rows, _lib.ptr(ws), rows, cols, IGNORE_INDEX, tag(logits.dtype),
              _lib.stream_of(logits))
    return loss, (logits, target, stats)


def cross_entropy_backward_from_saved(dloss: torch.Tensor, saved):
    logits, target, stats = saved
    _lib.require_gpu("cross_entropy_backward_from_saved", dloss, logits)
    if dloss.numel() != 1:
        raise ValueError(f"cross_entropy: dloss must hold one element, got {tuple(dloss.shape)}")
    if dloss.dtype != logits.dtype:
        dloss = dloss.to(logits.dtype)
    dloss = as_contiguous("dloss", dloss)
    rows, cols = logits.shape
    dlogits = torch.empty_like(logits)
    base = stats.data_ptr()
    _lib.call("eg_cross_entropy_bwd", _lib.ptr(dloss), _lib.ptr(logits), _lib.ptr(target), base,
              base + 4 * rows, _lib.ptr(dlogits), rows, cols, IGNORE_INDEX, tag(logits.dtype),
              _lib.stream_of(logits))
    return dlogits
