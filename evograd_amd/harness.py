"""Saved-state accounting and device timing for the autograd pairs.

``saved_bytes``/``describe_saved`` restate src/evograd/bench/harness.py:114-150
and ``saved_state_report`` restates src/evograd/bench/fair.py:297-322: logical
bytes over every saved tensor (inputs included), the bytes of the unique
storages behind them, and how much of that is input storage kept alive.

Timing follows the reference's fair protocol (src/evograd/bench/fair.py:338-440):
the Infinity Cache (256 MB MALL on MI355X) and L2 are flushed with a 512 MiB
write before each timed region, regions are bracketed by HIP events on the
current stream, and medians are reported.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass
from typing import Any, Callable

import torch


def normalize_saved(saved: Any) -> tuple:
    return tuple(saved) if isinstance(saved, (tuple, list)) else (saved,)


def saved_bytes(saved) -> int:
    return int(sum(t.numel() * t.element_size() for t in normalize_saved(saved)
                   if torch.is_tensor(t)))


def describe_saved(saved) -> list:
    out = []
    for v in normalize_saved(saved):
        if torch.is_tensor(v):
            out.append({"kind": "tensor", "shape": list(v.shape), "dtype": str(v.dtype),
                        "bytes": v.numel() * v.element_size()})
        else:
            out.append({"kind": "value", "type": type(v).__name__, "repr": repr(v)[:200]})
    return out


def saved_state_report(saved, values: dict) -> dict:
    inputs = {v.untyped_storage().data_ptr(): v.untyped_storage().nbytes()
              for v in values.values() if torch.is_tensor(v)}
    unique, retained = {}, {}
    logical = 0
    for v in normalize_saved(saved):
        if not torch.is_tensor(v):
            continue
        logical += v.numel() * v.element_size()
        st = v.untyped_storage()
        unique[st.data_ptr()] = st.nbytes()
        if st.data_ptr() in inputs:
            retained[st.data_ptr()] = inputs[st.data_ptr()]
    return {
        "logical_saved_bytes": logical,
        "unique_saved_storage_bytes": sum(unique.values()),
        "retained_input_bytes": sum(retained.values()),
        "new_storage_bytes": sum(unique.values()) - sum(retained.values()),
        "saved_tensors": describe_saved(saved),
    }


@dataclass(frozen=True)
class InputRecord:
    """What a candidate must leave unchanged in one input tensor: its identity
    (shape, strides, dtype, storage offset) always, its contents unless the
    declaration lets the backward overwrite it (``contents`` is None then)."""

    name: str
    identity: tuple
    contents: torch.Tensor | None


def _identity(t: torch.Tensor) -> tuple:
    return (tuple(t.shape), tuple(t.stride()), t.dtype, t.storage_offset())


def record_inputs(values: dict, may_overwrite: tuple = ()) -> tuple:
    """Record every tensor of a case (the rule of src/evograd/bench/fair.py:212-261)."""
    return tuple(InputRecord(name, _identity(v),
                             None if name in may_overwrite else v.detach().clone())
                 for name, v in values.items() if torch.is_tensor(v))


def check_inputs(values: dict, records: tuple, who: str) -> None:
    """Raise RuntimeError naming the first input whose identity or contents changed."""
    for rec in records:
        now = values[rec.name]
        if _identity(now) != rec.identity:
            raise RuntimeError(f"{who}: input {rec.name!r} changed from "
                               f"{rec.identity} to {_identity(now)} (shape, strides, "
                               "dtype, storage offset)")
        if rec.contents is not None and not torch.equal(now, rec.contents):
            raise RuntimeError(f"{who}: input {rec.name!r} was written to")


class CacheFlusher:
    """Writes a buffer larger than L2 + MALL so the next region starts cold."""

    def __init__(self, device, nbytes: int = 512 << 20):
        self.buf = torch.empty(nbytes // 4, dtype=torch.float32, device=device)

    def __call__(self):
        self.buf.fill_(1.0)


def time_regions(fn: Callable[[], Any], *, reps: int, warmup: int, flush: CacheFlusher | None,
                 setup: Callable[[], Any] | None = None) -> list:
    """Milliseconds of ``fn`` per rep, each bracketed by events on the current
    stream; ``setup`` (untimed) and the flush run before each region."""
    for _ in range(warmup):
        if setup is not None:
            setup()
        fn()
    torch.cuda.synchronize()
    samples = []
    stream = torch.cuda.current_stream()
    for _ in range(reps):
        if setup is not None:
            setup()
        if flush is not None:
            flush()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        fn()
        end.record(stream)
        end.synchronize()
        samples.append(start.elapsed_time(end))
    return samples


def summarize(samples: list) -> dict:
    s = sorted(samples)
    q = lambda f: s[min(len(s) - 1, max(0, int(round(f * (len(s) - 1)))))]
    return {"count": len(s), "median_ms": statistics.median(s), "q20_ms": q(0.2),
            "q80_ms": q(0.8), "min_ms": s[0]}
