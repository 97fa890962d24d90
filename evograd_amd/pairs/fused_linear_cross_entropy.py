"""Fused linear + cross entropy (FLCE) pair on gfx950.

Replaces fused_linear_cross_entropy_forward_ref
(src/evograd/ops/level2/fused_linear_cross_entropy/forward_ref.py:23-35: the mean
hard-label cross entropy of ``x @ weight.T`` against ``target``, ignore_index -100,
projection and logsumexp accumulated in fp32) under the contract of
fused_linear_cross_entropy/__init__.py:91-152: the ``[rows, vocab]`` logits are never
materialised in full, and neither is ``dlogits`` (its ``backward_semantics``: "dlogits
must not be materialized in full either"). One C entry point (``eg_flce_fwd``) runs
the whole pass on this library's kernels, one chunk of rows at a time: for 16-bit
inputs the MFMA logits product (``gemm.hip``) forms the softmax terms in its
epilogue (``exp(logit - group max)`` per 128-column group, with the group sums and
the target logit, all from the fp32 accumulators), one pass per row turns them into
the logsumexp, the row loss and the chunk's unit gradient ``softmax - onehot`` in
the input dtype, then ``dx_c = dl_c @ weight`` and ``dweight += dl_c.T @ x_c`` (the
product's epilogue adds the running sum in fp32), and at the end the mean loss.
fp32 inputs take fp32 logits chunks and separate logsumexp and gradient passes.

The gradient is formed in the forward because the backward's only input is the
scalar ``dloss``: the backward (``eg_scale_copy``) scales the saved unit gradients
by ``dloss / n_valid``. The loss is fp32, as the reference's forward returns it.
Saved state: ``(dx, dweight, n_valid)`` — the gradients in the inputs' dtypes and
one fp32 count, nothing of size rows x vocab.

Scratch (freed when the forward returns): the unit gradient of one chunk in the
input dtype, plus the group statistics of one chunk (16-bit inputs) or one chunk
of fp32 logits (fp32 inputs), and two fp32 values per row. By default a chunk holds
as many rows as 1 GiB of dlogits allows (4096 rows at the Llama-3 vocabulary in
bf16), so scratch grows with the chunk, not with rows x vocab. 16-bit inputs whose
hidden size is not a multiple of 64 (the product's k step) are copied into
zero-padded buffers first.
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
# Logits per chunk when set; None leaves the split to the library (chunk_rows 0):
# as many rows per chunk as 1 GiB of dlogits allows.
CHUNK_ELEMS = None


def chunk_rows(rows: int, vocab: int) -> int:
    """Rows per chunk passed to eg_flce_fwd: 0 (the library's default) unless
    CHUNK_ELEMS is set; then as many rows as CHUNK_ELEMS logits allow, rounded down
    to a power of two when that splits the rows."""
    if CHUNK_ELEMS is None:
        return 0
    rc = max(1, min(rows, CHUNK_ELEMS // max(vocab, 1)))
    if rc < rows:
        rc = 1 << (rc.bit_length() - 1)
    return rc


def _check(x, weight, target):
    _lib.require_gpu("fused_linear_cross_entropy", x, weight, target)
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError(f"fused_linear_cross_entropy: x {tuple(x.shape)} and weight "
                         f"{tuple(weight.shape)} must be [rows, hidden] and [vocab, hidden]")
    if target.dim() != 1 or target.shape[0] != x.shape[0]:
        raise ValueError(f"fused_linear_cross_entropy: target must be [rows]={x.shape[0]}, "
                         f"got {tuple(target.shape)}")
    if target.dtype != torch.int64:
        raise TypeError(f"fused_linear_cross_entropy: target must be int64, got {target.dtype}")
    if x.dtype != weight.dtype:
        raise TypeError(f"fused_linear_cross_entropy: x {x.dtype} and weight {weight.dtype} differ")
    tag(x.dtype)


def _pad_cols(t: torch.Tensor, cols: int) -> torch.Tensor:
    out = torch.zeros((t.shape[0], cols), dtype=t.dtype, device=t.device)
    out[:, :t.shape[1]] = t
    return out


def fused_linear_cross_entropy_forward_with_saved(x: torch.Tensor, weight: torch.Tensor,
                                                  target: torch.Tensor):
    _check(x, weight, target)
    x = as_contiguous("x", x)
    weight = as_contiguous("weight", weight)
    target = as_contiguous("target", target)
    rows, hidden = x.shape
    vocab = weight.shape[0]
    dt = x.dtype
    hp = hidden
    if dt != torch.float32 and hidden % 64:
        hp = (hidden + 63) // 64 * 64
        x, weight = _pad_cols(x, hp), _pad_cols(weight, hp)
    dx = torch.empty((rows, hp), dtype=dt, device=x.device)
    dw = torch.empty((vocab, hp), dtype=dt, device=x.device)
    out = torch.empty(2, dtype=torch.float32, device=x.device)  # loss | n_valid
    rc = chunk_rows(rows, vocab)
    ws = workspace(_lib.query("eg_flce_workspace_bytes", rows, hp, vocab, rc, tag(dt)), x.device)
    _lib.call("eg_flce_fwd", _lib.ptr(x), _lib.ptr(weight), _lib.ptr(target), out.data_ptr(),
              _lib.ptr(dx), _lib.ptr(dw), out[1:].data_ptr(), _lib.ptr(ws), rows, hp, vocab,
              IGNORE_INDEX, rc, tag(dt), _lib.stream_of(x))
    del ws
    if hp != hidden:
        dx, dw = dx[:, :hidden].contiguous(), dw[:, :hidden].contiguous()
    loss = out[0].clone()
    return loss, (dx, dw, out[1:].clone())


def fused_linear_cross_entropy_backward_from_saved(dloss: torch.Tensor, saved):
    dx_u, dw_u, n_valid = saved
    _lib.require_gpu("fused_linear_cross_entropy_backward_from_saved", dloss, dx_u)
    if dloss.numel() != 1:
        raise ValueError(f"fused_linear_cross_entropy: dloss must hold one element, "
                         f"got {tuple(dloss.shape)}")
    dloss = as_contiguous("dloss", dloss)
    stream = _lib.stream_of(dx_u)
    outs = []
    for g in (dx_u, dw_u):
        o = torch.empty_like(g)
        _lib.call("eg_scale_copy", g.data_ptr(), tag(g.dtype), o.data_ptr(), tag(o.dtype),
                  g.numel(), dloss.data_ptr(), tag(dloss.dtype), n_valid.data_ptr(), stream)
        outs.append(o)
    return tuple(outs)
