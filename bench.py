#!/usr/bin/env python3
"""Benchmark of the autograd-pair hot path on one MI355X.

Metric: fwd+bwd step latency (us) + % HBM/MFMA roofline per op;
saved bytes vs CPU. The headline ``value`` is the full-step (forward + backward)
latency of RMSNorm bf16 x[16384, 4096], eps 1e-6; every other
BASELINE configuration is measured the same way and reported under ``ops``, with the
operators beyond BASELINE at their declared benchmark workloads. ``op@label``
selects another labelled benchmark workload of an operator (``softmax@vocab``: bf16
rows of the Llama-3 vocabulary, the reference's timed default width).

A step is one forward_with_saved + backward_from_saved of the HIP pair over
synthetic seeded inputs already resident in HBM. Before every timed region a
512 MiB write evicts L2 and the 256 MB Infinity Cache; each region is bracketed
by HIP events on torch's current stream, which is the stream the library
launches on. ``steps`` regions are timed per phase after ``warmup`` untimed ones
and medians are reported.

The CPU baseline is the reference's eager PyTorch autograd path (the oracle
package's restated forwards, fused ``F.rms_norm``/``F.layer_norm`` where the
reference declares a runtime forward, ``F.scaled_dot_product_attention`` for
attention) timed on this host's cores: the whole workload for the memory-bound
operators, a bounded head/row sample scaled to the full workload for attention
and the fused linear cross entropy, and the T=1024 layer scaled by model FLOPs
for the larger layers.

The decoder layer (``llama3_decoder_layer``) is timed at the reference's grid, B=1 and
T in {1024, 2048, 4096} at Llama-3-8B widths, with its MFMA fraction over the
layer's model FLOPs. ``sweeps`` holds the memory-bound operators over the
reference's token sweeps (src/evograd/opdecl/models.py:286, :293).

Each operator with an eager spelling also reports ``gpu_eager_full_us``: the reference's
eager forward (torch operators) plus torch autograd on the same GPU and inputs, and
``speedup_vs_gpu_eager``. ``sustained`` holds the device's sustained MFMA and copy rates
measured in the same run.

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--ops a,b] [--no-cpu]
                       [--no-sweep] [--no-eager]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd step latency (us) + % HBM/MFMA roofline per op; saved bytes vs CPU"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/CU/clk
HEADLINE = "rmsnorm"
LAYER = "llama3_decoder_layer"
ALL_OPS = ("softmax", "rmsnorm", "layernorm", "swiglu", "rope", "causal_attention",
           "fused_add_rms_norm", "causal_attention_gqa", "llama3_attention", "cross_entropy",
           "fused_linear_cross_entropy", "softmax@vocab", f"{LAYER}@llama3_8b_T1024",
           f"{LAYER}@llama3_8b_T2048", f"{LAYER}@llama3_8b_T4096")
# The reference's timed token sweeps (src/evograd/opdecl/models.py:286, :293): the
# residual-stream and MLP operators over LLAMA_TOKEN_SWEEP, the vocabulary-width
# ones over LLAMA_VOCAB_TOKEN_SWEEP.
LLAMA_TOKEN_SWEEP = (1024, 2048, 4096, 8192, 16384)
LLAMA_VOCAB_TOKEN_SWEEP = (512, 1024, 2048, 4096, 8192)
# Two points below the reference's sweep for the norms with a shape dispatcher: there
# its small-shape program runs the one-launch backward (up to 512 rows).
SMALL_NORM_POINTS = (256, 512)
SWEEP_OPS = {
    "rmsnorm": SMALL_NORM_POINTS + LLAMA_TOKEN_SWEEP,
    "layernorm": SMALL_NORM_POINTS + LLAMA_TOKEN_SWEEP, "swiglu": LLAMA_TOKEN_SWEEP,
    "fused_add_rms_norm": LLAMA_TOKEN_SWEEP, "rope": LLAMA_TOKEN_SWEEP,
    "cross_entropy": LLAMA_VOCAB_TOKEN_SWEEP, "softmax@vocab": LLAMA_VOCAB_TOKEN_SWEEP,
}
# Operators whose CPU step at the full benchmark size costs a few hundred ms to about
# a second on the host cores: their CPU baseline runs the whole workload.
CPU_FULL = ("softmax", "rmsnorm", "layernorm", "swiglu", "fused_add_rms_norm", "rope",
            "cross_entropy", "softmax@vocab")


def split_name(name: str) -> tuple:
    """``op`` or ``op@label``: the operator and the label of its benchmark workload
    (the first benchmark workload when no label is given)."""
    base, _, label = name.partition("@")
    return base, label


def bench_workload(op, label: str):
    if not label:
        return op.benchmark[0]
    for w in op.benchmark:
        if w.label == label:
            return w
    raise KeyError(f"{op.name} has no benchmark workload labelled {label!r}")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------ algorithmic work
def algorithmic_work(name: str, w, extra_k_heads: int = 0) -> dict:
    """Bytes (memory-bound ops) or FLOPs (attention) per forward and backward,
    counting each tensor the op must read or write exactly once."""
    d = w.dims
    es = {"float32": 4, "float16": 2, "bfloat16": 2}[w.dtype]
    if name == "softmax":
        n = d["rows"] * d["cols"] * es
        return {"unit": "bytes", "fwd": 2 * n, "bwd": 3 * n}
    if name == "rmsnorm":
        R, H = d["rows"], d["hidden"]
        n = R * H * es
        return {"unit": "bytes", "fwd": 2 * n + H * es + 4 * R,
                "bwd": 3 * n + 4 * R + 2 * H * es}
    if name == "layernorm":
        R, H = d["rows"], d["hidden"]
        n = R * H * es
        return {"unit": "bytes", "fwd": 2 * n + 2 * H * es + 8 * R,
                "bwd": 3 * n + 8 * R + 3 * H * es}
    if name == "swiglu":
        n = d["rows"] * d["cols"] * es
        return {"unit": "bytes", "fwd": 3 * n, "bwd": 5 * n}
    if name == "fused_add_rms_norm":
        # fwd reads x, r, weight and writes out, rstd; bwd reads dout and the
        # saved x, r, weight, rstd and writes the one gradient through s (returned
        # as dx and dr) and dweight.
        R, C = d["rows"], d["cols"]
        n = R * C * es
        return {"unit": "bytes", "fwd": 3 * n + C * es + 4 * R,
                "bwd": 4 * n + 4 * R + 2 * C * es}
    if name == "cross_entropy":
        # fwd reads logits and target once and writes lse and the loss; bwd reads
        # logits, target and lse and writes dlogits.
        R, C = d["rows"], d["cols"]
        n = R * C * es
        return {"unit": "bytes", "fwd": n + 8 * R + 4 * R + es, "bwd": 2 * n + 8 * R + 4 * R}
    if name == "fused_linear_cross_entropy":
        # three rows x hidden x vocab products, all in the forward (the backward
        # only scales the saved gradients)
        R, Hd, V = d["rows"], d["hidden"], d["vocab"]
        return {"unit": "flops", "fwd": 3 * 2.0 * R * Hd * V, "bwd": 0.0}
    if name == "rope":
        B, H, T, D = d["B"], d["n_heads"], d["T"], d["head_dim"]
        xb = B * (H + extra_k_heads) * T * D * es
        tables = 2 * T * D * 4
        return {"unit": "bytes", "fwd": 2 * xb + tables, "bwd": 2 * xb + tables}
    if name in ("causal_attention", "causal_attention_gqa", "llama3_attention"):
        B, H, S, D = d["B"], d["H"], d["S"], d["D"]  # FLOPs count query heads
        dense = 2.0 * S * S * D * B * H  # one S x S x D product
        return {"unit": "flops", "fwd": 2 * dense / 2, "bwd": 5 * dense / 2}
    if name == LAYER:
        # model FLOPs: the seven projections (2 M P forward, 4 M P backward for P
        # weights) and the causal attention (FlashAttention convention); the
        # recomputed projections of the backward are not counted
        return {"unit": "flops", **layer_flops(d)}
    raise KeyError(name)


def flce_chunk_rows(d: dict) -> int:
    """Rows per chunk of eg_flce_fwd's default split for 16-bit inputs: as many as
    1 GiB of dlogits rows (the vocabulary padded to 64) allows, a multiple of 256."""
    vp = (d["vocab"] + 63) // 64 * 64
    rc = (1 << 30) // (vp * 2)
    if rc >= d["rows"]:
        return d["rows"]
    return rc // 256 * 256 if rc >= 256 else 1 << (rc.bit_length() - 1)


def layer_flops(d: dict) -> dict:
    M = d["B"] * d["T"]
    hid, qo, kvo, inter = d["hidden"], d["q_out"], d["kv_out"], d["intermediate"]
    P = hid * (qo + 2 * kvo) + qo * hid + 3 * hid * inter
    dense = 2.0 * d["T"] * d["T"] * d["head_dim"] * d["B"] * (qo // d["head_dim"])
    return {"fwd": 2.0 * M * P + dense, "bwd": 4.0 * M * P + 5 * dense / 2}


# The kernel whose roofline each op reports: (phase, kernel name, occurrence of that
# name among the phase's launches), with its algorithmic work per launch from
# dominant_work. Launch sequences are discovered by the timing hook (every launch
# of a phase is timed and named), so split products and chunk loops need no list.
DOMINANT = {
    "softmax": ("bwd", "softmax_bwd_reg", 0), "rmsnorm": ("bwd", "norm_bwd_ring", 0),
    "layernorm": ("bwd", "norm_bwd_ring", 0), "swiglu": ("bwd", "swiglu_bwd_kernel", 0),
    "rope": ("fwd", "rope_kernel", 0), "causal_attention": ("bwd", "attn_dkdv_kernel", 0),
    "fused_add_rms_norm": ("bwd", "norm_bwd_ring", 0),
    "causal_attention_gqa": ("bwd", "attn_dkdv_kernel", 0),
    "llama3_attention": ("bwd", "attn_dkdv_kernel", 0),
    "cross_entropy": ("bwd", "xent_bwd_flat_kernel", 0),
    # eg_flce_fwd at 8192 rows of 128256 (bf16: two chunks of 4096 rows, 1 GiB of
    # dlogits each): per chunk the logits product (softmax epilogue), the fix-up,
    # the dx product and the dweight product; the last chunk's dweight product
    # (adding the fp32 sum of the first) is the 6th product
    "fused_linear_cross_entropy": ("fwd", "gemm_kernel", 5),
    # bf16 rows of 128256: the backward's y held in registers as raw packs
    "softmax@vocab": ("bwd", "softmax_bwd_lds", 0),
    # the decoder layer's gate and up projections, one product over the segmented
    # weights [Wg; Wu]: its 3rd product (after [q | k | v] and o)
    **{f"{LAYER}@llama3_8b_T{t}": ("fwd", "gemm_kernel", 2) for t in (1024, 2048, 4096)},
}


def dominant_work(name: str, w, work: dict) -> float:
    """Algorithmic bytes (or FLOPs) of one launch of the op's dominant kernel."""
    d = w.dims
    es = {"float32": 4, "float16": 2, "bfloat16": 2}[w.dtype]
    if name == "fused_linear_cross_entropy":
        # the last chunk's dweight product: dlogits_c.T @ x_c over its rows
        return 2.0 * flce_chunk_rows(d) * d["hidden"] * d["vocab"]
    if name == "rmsnorm":  # the column sum writes dweight
        return work["bwd"] - d["hidden"] * es
    if name == "fused_add_rms_norm":
        return work["bwd"] - d["cols"] * es
    if name == "layernorm":  # the column sum writes dweight and dbias
        return work["bwd"] - 2 * d["hidden"] * es
    if name in ("causal_attention", "causal_attention_gqa", "llama3_attention"):
        # dK/dV kernel: S, dP, dV, dK of the five products
        return work["bwd"] * 4 / 5
    if name == LAYER:  # the gate and up projections as one product h2 [Wg; Wu]^T
        return 2.0 * d["B"] * d["T"] * d["hidden"] * 2 * d["intermediate"]
    phase = DOMINANT[name][0]
    return work[phase]


def kernel_times(name: str, fwd, bwd_call, setup_bwd, state, flush, steps: int) -> dict:
    """Median microseconds of every kernel of the forward and backward calls, each
    timed by events the dispatch records (evograd_amd.timing) on a cold cache, keyed
    "phase:index:kernel". Launches are numbered from 0 until an armed index is not
    reached."""
    import torch

    from evograd_amd.timing import KernelTimer

    timer = KernelTimer()
    out = {}
    try:
        for phase in ("fwd", "bwd"):
            for idx in range(512):
                samples, label = [], ""
                for _ in range(steps):
                    if phase == "bwd":
                        setup_bwd()
                    flush()
                    timer.arm(idx)
                    if phase == "fwd":
                        fwd()
                    else:
                        bwd_call(state["saved"])
                    label = timer.label()
                    if not label:  # the phase launches fewer kernels
                        timer.fired()
                        break
                    samples.append(timer.elapsed_ms() * 1e3)
                if not samples:
                    break
                out[f"{phase}:{idx}:{label}"] = statistics.median(samples)
        torch.cuda.synchronize()
    finally:
        timer.close()
    return out


def find_kernel(kt: dict, phase: str, kname: str, occurrence: int) -> str:
    """Key of the occurrence-th launch of kernel kname in a phase."""
    hits = [k for k in kt if k.split(":")[0] == phase and k.split(":")[2] == kname]
    if len(hits) <= occurrence:
        raise KeyError(f"{phase} has {len(hits)} launches of {kname}, not {occurrence + 1}")
    return hits[occurrence]


# ----------------------------------------------------------------- GPU side
def gpu_op(name: str, steps: int, warmup: int, flush) -> dict:
    import torch

    from evograd_amd import decls, pair_module
    from evograd_amd.bind import backward_inactive_kwargs, bind, lookup_pair
    from evograd_amd.harness import saved_state_report, summarize, time_regions
    from evograd_amd.inputs import make_case_inputs

    base, label = split_name(name)
    op = decls.get_op(base)
    mod = pair_module(base)
    w = bench_workload(op, label)
    inputs = make_case_inputs(op, w, "cuda")
    k_heads = 0
    if name == "rope":
        # joint q/k launch: q [B, 32, T, D] from the declared recipe, k [B, 8, T, D]
        k_heads = int(w.extra["k_heads"])
        q = inputs["x"]
        torch.manual_seed(w.dims["T"] * 100003 + k_heads * 1009 + w.dims["head_dim"])
        k = torch.randn((q.shape[0], k_heads, q.shape[2], q.shape[3]), device="cuda",
                        dtype=q.dtype)
        dk = torch.randn_like(k)
        cos, sin = inputs["cos"], inputs["sin"]
        fwd = lambda: mod.rope_qk_forward_with_saved(q, k, cos, sin)  # noqa: E731
        bwd_call = lambda saved: mod.rope_qk_backward_from_saved((inputs["dy"], dk), saved)  # noqa: E731
        values = {"q": q, "k": k, "cos": cos, "sin": sin}
        q_leaf, k_leaf = q.detach().requires_grad_(True), k.detach().requires_grad_(True)

        def autograd_fn():
            q_leaf.grad = k_leaf.grad = None
            qo, ko = mod.RopeQK.apply(q_leaf, k_leaf, cos, sin)
            torch.autograd.backward((qo, ko), (inputs["dy"], dk))
    else:
        f, b = lookup_pair(op, mod)
        args = [inputs.get(a.name, getattr(a, "default", None)) for a in op.args]
        kw = backward_inactive_kwargs(op, b, inputs)
        dy = inputs[op.upstream_grad_name]
        fwd = lambda: f(*args)  # noqa: E731
        bwd_call = lambda saved: b(dy, saved, **kw)  # noqa: E731
        values = {a.name: inputs[a.name] for a in op.args if a.name in inputs}
        bound = bind(op, mod)
        leaves = [a.detach().requires_grad_(True) if torch.is_tensor(a) and a.is_floating_point()
                  and isinstance(spec, decls.Active) else a
                  for a, spec in zip(args, op.args)]

        def autograd_fn():
            for lf in leaves:
                if torch.is_tensor(lf):
                    lf.grad = None
            y = bound(*leaves)
            y.backward(dy)

    with torch.no_grad():
        _, saved = fwd()
        report = saved_state_report(saved, values)
    state = {}

    def setup_bwd():
        state["saved"] = fwd()[1]

    fwd_ms = time_regions(fwd, reps=steps, warmup=warmup, flush=flush)
    bwd_ms = time_regions(lambda: bwd_call(state["saved"]), reps=steps, warmup=warmup,
                          flush=flush, setup=setup_bwd)
    full_ms = time_regions(lambda: bwd_call(fwd()[1]), reps=steps, warmup=warmup, flush=flush)
    ag = None
    if autograd_fn is not None:
        ag = summarize(time_regions(autograd_fn, reps=steps, warmup=warmup, flush=flush))
    work = algorithmic_work(base, w, k_heads)
    kt = kernel_times(name, fwd, bwd_call, setup_bwd, state, flush, steps)
    sf, sb, sfull = summarize(fwd_ms), summarize(bwd_ms), summarize(full_ms)
    out = {
        "config": {"dims": w.dims, "dtype": w.dtype, **({"k_heads": k_heads} if k_heads else {})},
        "fwd_us": sf["median_ms"] * 1e3,
        "bwd_us": sb["median_ms"] * 1e3,
        "full_us": sfull["median_ms"] * 1e3,
        "full_q20_us": sfull["q20_ms"] * 1e3,
        "full_q80_us": sfull["q80_ms"] * 1e3,
        "autograd_full_us": ag["median_ms"] * 1e3 if ag else None,
        "saved": {k: v for k, v in report.items() if k != "saved_tensors"},
        "saved_tensors": report["saved_tensors"],
        "kernels_us": kt,
    }
    if base == "fused_linear_cross_entropy":
        # the forward's scratch (one chunk of dlogits and group statistics, the fp32
        # dweight sum over chunks), freed when the forward returns
        from evograd_amd import _lib
        from evograd_amd.pairs._util import tag

        d = w.dims
        out["saved"]["peak_scratch_bytes"] = int(_lib.query(
            "eg_flce_workspace_bytes", d["rows"], d["hidden"], d["vocab"], 0,
            tag(inputs["x"].dtype)))
    phase, kname, occurrence = DOMINANT[name]
    kkey = find_kernel(kt, phase, kname, occurrence)
    k_us = kt[kkey]
    k_work = dominant_work(base, w, work)
    k_unit = work["unit"]
    if k_unit == "bytes":
        k_rate = k_work / (k_us * 1e-6) / 1e9
        out["dominant_kernel"] = {"name": kkey, "phase": phase, "us": k_us, "bytes": k_work,
                                  "achieved_gbs": k_rate, "frac": k_rate / HBM_PEAK_GBS}
    else:
        k_rate = k_work / (k_us * 1e-6) / 1e12
        out["dominant_kernel"] = {"name": kkey, "phase": phase, "us": k_us, "flops": k_work,
                                  "achieved_tflops": k_rate, "frac": k_rate / BF16_PEAK_TFLOPS}
    mem_inputs = sum(values[n].numel() * values[n].element_size()
                     for n in op.memory_input_names() if n in values and torch.is_tensor(values[n]))
    out["saved"]["ratio_to_memory_inputs"] = (report["logical_saved_bytes"] / mem_inputs
                                              if mem_inputs else None)
    if work["unit"] == "bytes":
        for phase, ms in (("fwd", sf["median_ms"]), ("bwd", sb["median_ms"])):
            out[f"{phase}_gbs"] = work[phase] / (ms * 1e-3) / 1e9
        full_gbs = (work["fwd"] + work["bwd"]) / (sfull["median_ms"] * 1e-3) / 1e9
        out.update(algorithmic_bytes=work, full_gbs=full_gbs,
                   hbm_frac_full=full_gbs / HBM_PEAK_GBS,
                   hbm_frac_bwd=out["bwd_gbs"] / HBM_PEAK_GBS)
    else:
        for phase, ms in (("fwd", sf["median_ms"]), ("bwd", sb["median_ms"])):
            out[f"{phase}_tflops"] = work[phase] / (ms * 1e-3) / 1e12
        full_tf = (work["fwd"] + work["bwd"]) / (sfull["median_ms"] * 1e-3) / 1e12
        out.update(algorithmic_flops=work, full_tflops=full_tf,
                   mfma_frac_full=full_tf / BF16_PEAK_TFLOPS)
    del inputs, saved, state
    torch.cuda.empty_cache()
    return out


def sweep_op(name: str, tokens: tuple, steps: int, warmup: int, flush) -> dict:
    """Full-step latency (forward + backward, cold cache, median) and the HBM
    fraction of an operator at each token count of the reference's sweep, the
    other dims at the benchmark workload's (RoPE: one q tensor of 32 heads, B=1)."""
    import dataclasses

    import torch

    from evograd_amd import DISPATCH_MODULES, decls, dispatch_module, pair_module
    from evograd_amd.bind import backward_inactive_kwargs, lookup_pair
    from evograd_amd.harness import summarize, time_regions
    from evograd_amd.inputs import make_case_inputs

    base, label = split_name(name)
    op = decls.get_op(base)
    f, b = lookup_pair(op, pair_module(base))
    # with a shape dispatcher (small-shape program below the regime split), the
    # dispatched pair is timed too
    disp = None
    if base in DISPATCH_MODULES and not label:
        disp = lookup_pair(op, dispatch_module(base))
    w0 = bench_workload(op, label)
    out = {}
    for t in tokens:
        if base == "rope":
            dims = dict(w0.dims, B=1, T=t)
        else:
            dims = dict(w0.dims, rows=t)
        w = dataclasses.replace(w0, dims=dims)
        inputs = make_case_inputs(op, w, "cuda")
        args = [inputs.get(a.name, getattr(a, "default", None)) for a in op.args]
        kw = backward_inactive_kwargs(op, b, inputs)
        dy = inputs[op.upstream_grad_name]
        ms = summarize(time_regions(lambda: b(dy, f(*args)[1], **kw), reps=steps,
                                    warmup=warmup, flush=flush))["median_ms"]
        work = algorithmic_work(base, w)
        gbs = (work["fwd"] + work["bwd"]) / (ms * 1e-3) / 1e9
        state = {}

        def setup_bwd():
            state["saved"] = f(*args)[1]

        kt = kernel_times(name, lambda: f(*args), lambda saved: b(dy, saved, **kw), setup_bwd,
                          state, flush, max(3, steps // 2))
        out[str(t)] = {"full_us": round(ms * 1e3, 2), "hbm_frac_full": round(gbs / HBM_PEAK_GBS, 4),
                       "kernels_us": {k: round(v, 2) for k, v in kt.items()}, "dims": dims}
        if disp is not None:
            df, db = disp
            dms = summarize(time_regions(lambda: db(dy, df(*args)[1], **kw), reps=steps,
                                         warmup=warmup, flush=flush))["median_ms"]
            dgbs = (work["fwd"] + work["bwd"]) / (dms * 1e-3) / 1e9
            out[str(t)].update(dispatch_full_us=round(dms * 1e3, 2),
                               dispatch_hbm_frac_full=round(dgbs / HBM_PEAK_GBS, 4),
                               dispatch_route=int(df(*args)[1][0]))
        del inputs, args, dy
        torch.cuda.empty_cache()
    return out


# ----------------------------------------------------------------- CPU side
def cpu_baseline(name: str) -> dict:
    """Eager PyTorch autograd on the host cores over a bounded sample, scaled."""
    import torch

    from evograd_amd import decls
    from evograd_amd.inputs import make_case_inputs
    from evograd_amd.opdecl import shape_tokens
    from oracle.oracle import check_runtime_forward, resolve_runtime_forward

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    name, label = split_name(name)
    op = decls.get_op(name)
    w = bench_workload(op, label)
    d = w.dims
    # The sample: leading slices of the benchmark's own GPU-seeded tensors.
    full_name = name + (f"@{label}" if label else "")
    if full_name in CPU_FULL:
        cut, scale = {}, 1.0
        sample = "full workload"
        if name == "rope":
            # q [B, n_heads, T, D] of the declared recipe; the joint launch's k heads
            # are the same computation on B * k_heads more rows
            full = d["B"] * (d["n_heads"] + int(w.extra["k_heads"]))
            scale = full / (d["B"] * d["n_heads"])
            sample = (f"full q [{d['B']}, {d['n_heads']}, {d['T']}, {d['head_dim']}], scaled "
                      f"x{scale:g} for the k heads of the joint q/k workload")
    elif name == LAYER:
        # the first 1024 tokens (the whole T=1024 workload), scaled by model FLOPs
        t = min(d["T"], 1024)
        cut = {"T": t}
        small = dict(d, T=t)
        f_full, f_small = layer_flops(d), layer_flops(small)
        scale = (f_full["fwd"] + f_full["bwd"]) / (f_small["fwd"] + f_small["bwd"])
        sample = ("full workload" if t == d["T"] else
                  f"first {t} of {d['T']} tokens, scaled x{scale:.3g} by model FLOPs")
    elif name == "fused_linear_cross_entropy":
        cut = {"rows": 64}
        scale = d["rows"] / 64
        sample = f"first 64 of {d['rows']} rows"
    elif name in ("causal_attention_gqa", "llama3_attention"):
        # kv head 0 of batch 0 and its group of query heads
        full = d["B"] * d["KVH"]
        cut = {"B": 1, "KVH": 1, "H": d["H"] // d["KVH"]}
        scale = float(full)
        sample = f"1 of {full} (batch, kv head) groups of {cut['H']} query heads"
    else:
        full = d["B"] * d["H"]
        cut = {"B": 1, "H": 1}
        scale = float(full)
        sample = f"1 of {full} (batch, head) pairs"
    checked = check_runtime_forward(op, "cpu")
    shapes = {a.name: a.shape for a in op.args if getattr(a, "shape", None)}
    shapes[op.upstream_grad_name] = op.output.shape
    inputs = {}
    for key, value in make_case_inputs(op, w, "cuda").items():
        tokens = shape_tokens(shapes.get(key))
        if torch.is_tensor(value):
            if tokens:
                value = value[tuple(slice(0, cut[t]) if t in cut else slice(None)
                                    for t in tokens)]
            value = value.detach().to("cpu").contiguous()
        inputs[key] = value
    torch.cuda.empty_cache()
    fwd = resolve_runtime_forward(op)
    args = []
    leaves = []
    for a in op.args:
        v = inputs.get(a.name, getattr(a, "default", None))
        if isinstance(a, decls.Active):
            v = v.detach().requires_grad_(True)
            leaves.append(v)
        args.append(v)
    dy = inputs[op.upstream_grad_name]

    def step():
        for lf in leaves:
            lf.grad = None
        y = fwd(*args)
        y.backward(dy)

    step()
    samples = []
    t_end = time.perf_counter() + 10.0
    while len(samples) < 3 or (len(samples) < 7 and time.perf_counter() < t_end):
        t0 = time.perf_counter_ns()
        step()
        samples.append((time.perf_counter_ns() - t0) / 1e3)
    us = statistics.median(samples) * scale
    verified = (f"runtime forward held to {op.forward} on {checked} correctness workloads"
                if checked else "the declared forward itself")
    how = (f"{len(samples)} reps, median" if scale == 1.0 else
           f"{len(samples)} reps, median scaled x{scale:.4g} to the full workload")
    return {"value": us, "unit": "us", "cores": cores, "kind": "port",
            "sample": f"{sample} of the benchmark's GPU-seeded inputs copied to the host, {how}",
            "timed_forward": f"{op.runtime_forward or op.forward} ({verified})",
            "what": f"eager torch autograd on CPU of {op.runtime_forward or op.forward}"}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ------------------------------------------------------ eager torch on this GPU
# The reference's eager spellings of each forward (its runtime forwards where it
# declares one), written here with torch's own operators, run through torch
# autograd on the same GPU and inputs: what a user of the reference gets without
# these kernels. Attention goes through F.scaled_dot_product_attention limited to
# its flash and memory-efficient backends (never the math backend's batched
# products); the decoder layer and the RoPE -> attention pair are not timed.
EAGER_OPS = ("softmax", "rmsnorm", "layernorm", "swiglu", "rope", "fused_add_rms_norm",
             "causal_attention", "causal_attention_gqa", "cross_entropy",
             "fused_linear_cross_entropy", "softmax@vocab")


def _eager_forward(name: str):
    import torch
    import torch.nn.functional as F

    def rotate_half(x):
        h = x.shape[-1] // 2
        return torch.cat((-x[..., h:], x[..., :h]), dim=-1)

    def sdpa(q, k, v):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True)

    def gqa(q, k, v):
        r = q.shape[1] // k.shape[1]
        if r > 1:
            k, v = k.repeat_interleave(r, dim=1), v.repeat_interleave(r, dim=1)
        return sdpa(q, k, v)

    return {
        # softmax/forward_ref.py:6-7
        "softmax": lambda x: torch.softmax(x.float(), dim=-1).to(x.dtype),
        # rmsnorm/forward_ref.py:24-34, layernorm/forward_ref.py:26-42 (runtime forwards)
        "rmsnorm": lambda x, w, eps: F.rms_norm(x, (x.shape[-1],), weight=w, eps=eps),
        "layernorm": lambda x, w, b, eps: F.layer_norm(x, (x.shape[-1],), weight=w, bias=b,
                                                       eps=eps),
        # swiglu/forward_ref.py:6-9
        "swiglu": lambda a, b: F.silu(a.float()).to(a.dtype) * b,
        # rope/forward_ref.py:28-47
        "rope": lambda x, c, s: (x.float() * c[None, None].float()
                                 + rotate_half(x.float()) * s[None, None].float()).to(x.dtype),
        # fused_add_rms_norm/forward_ref.py:19-34
        "fused_add_rms_norm": lambda x, r, w, eps: F.rms_norm(x + r, (x.shape[-1],), weight=w,
                                                              eps=eps),
        # llama3_decoder_layer/forward_ref.py:101-107
        "causal_attention": sdpa,
        "causal_attention_gqa": gqa,
        # cross_entropy/forward_ref.py:6-12
        "cross_entropy": lambda lg, t: F.cross_entropy(lg.float(), t).to(lg.dtype),
        # fused_linear_cross_entropy/forward_ref.py:23-35
        "fused_linear_cross_entropy": lambda x, w, t: F.cross_entropy(
            torch.matmul(x.float(), w.float().t()), t),
    }[name]


def gpu_eager(name: str, steps: int, warmup: int, flush) -> dict:
    """Full step (forward + autograd backward) of the eager spelling on this GPU,
    timed like the pairs: cache flush, events around each step, median."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from evograd_amd import decls
    from evograd_amd.inputs import make_case_inputs

    base, label = split_name(name)
    op = decls.get_op(base)
    w = bench_workload(op, label)
    inputs = make_case_inputs(op, w, "cuda")
    fwd = _eager_forward(base)
    args, leaves = [], []
    for a in op.args:
        v = inputs.get(a.name, getattr(a, "default", None))
        if isinstance(a, decls.Active):
            v = v.detach().requires_grad_(True)
            leaves.append(v)
        args.append(v)
    dy = inputs[op.upstream_grad_name]

    def step():
        for lf in leaves:
            lf.grad = None
        fwd(*args).backward(dy)

    scale, note = 1.0, ""
    if base == "rope":  # q of the joint q/k workload; its k heads are the same computation
        scale = (w.dims["n_heads"] + int(w.extra["k_heads"])) / w.dims["n_heads"]
        note = f"q timed, scaled x{scale:g} for the k heads"
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        samples = []
        for _ in range(steps):
            flush()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            step()
            e1.record()
            e1.synchronize()
            samples.append(e0.elapsed_time(e1) * 1e3)
    del inputs, args, leaves, dy
    torch.cuda.empty_cache()
    out = {"full_us": round(statistics.median(samples) * scale, 2)}
    if note:
        out["note"] = note
    return out


# ------------------------------------------------------------ sustained rates
PROBE_ITERS = 100000   # about 0.1 s per probe launch


def sustained_rates(reps: int = 3) -> dict:
    """The device's sustained rates in this run, beside the published peaks: bf16
    MFMA from registers on random operands (eg_probe_mfma_bf16, one 256-thread
    workgroup per CU, launches of about 0.1 s so power management settles), the same
    work as v_mfma_f32_16x16x32_bf16 at two waves per SIMD, the 32 x 32 x 16 work fed
    by one 1 KiB LDS operand read per MFMA (the attention kernels' operand traffic),
    without and with one exponential per MFMA (eg_probe_mfma_mix kinds 1-3), and an
    HBM copy (torch's copy kernel over 1 GiB each way, larger than every cache)."""
    import torch

    from evograd_amd import _lib

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device="cuda").manual_seed(7)
    operands = torch.randn(16384, device="cuda", generator=g).to(torch.bfloat16)  # 32 KiB
    out = torch.empty(2 * cus * 256, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def probe(iters):
        _lib.call("eg_probe_mfma_bf16", operands.data_ptr(), out.data_ptr(), cus, iters, stream)

    def mix(kind, iters):
        _lib.call("eg_probe_mfma_mix", kind, operands.data_ptr(), out.data_ptr(), 2 * cus, iters,
                  stream)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e-3)
        return statistics.median(ts)

    probe(PROBE_ITERS // 10)
    s = timed(lambda: probe(PROBE_ITERS))
    if not torch.isfinite(out[: cus * 256]).all():
        raise RuntimeError("MFMA probe produced non-finite checksums")
    mfma_tflops = cus * 4 * PROBE_ITERS * 64 * 32768 / s / 1e12
    kinds = {}
    for kind, key in ((1, "mfma16_bf16_tflops"), (2, "mfma_lds_operand_tflops"),
                      (3, "mfma_lds_operand_exp_tflops")):
        it = PROBE_ITERS // 2
        t = timed(lambda: mix(kind, it))
        if not torch.isfinite(out).all():
            raise RuntimeError(f"MFMA probe kind {kind} produced non-finite checksums")
        kinds[key] = round(2 * cus * 4 * it * 64 * 32768 / t / 1e12, 1)
    n = 1 << 29  # bf16 elements: 1 GiB
    src = torch.randn(n, device="cuda", generator=g, dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    c = timed(lambda: dst.copy_(src))
    copy_gbs = 2 * n * 2 / c / 1e9
    del src, dst
    torch.cuda.empty_cache()
    res = {
        "mfma_bf16_tflops": round(mfma_tflops, 1),
        "mfma_frac_of_peak": round(mfma_tflops / BF16_PEAK_TFLOPS, 4),
    }
    for key, v in kinds.items():
        res[key] = v
        res[key.replace("_tflops", "_frac_of_peak")] = round(v / BF16_PEAK_TFLOPS, 4)
    res.update({
        "hbm_copy_gbs": round(copy_gbs, 1),
        "hbm_copy_frac_of_peak": round(copy_gbs / HBM_PEAK_GBS, 4),
        "how": ("eg_probe_mfma_bf16: 64 v_mfma_f32_32x32x16_bf16 per wave per iteration from "
                f"registers, random bf16 operands, {cus} workgroups x {PROBE_ITERS} iterations; "
                "eg_probe_mfma_mix kinds 1-3 (the same FLOPs as 16x16x32 from registers; as "
                "32x32x16 each fed one 1 KiB ds_read_b128; the latter plus one exp per MFMA), "
                f"{2 * cus} workgroups (two waves per SIMD) x {PROBE_ITERS // 2} iterations; "
                f"medians of {reps}; copy: torch copy_ of 1 GiB bf16, median of {reps}"),
    })
    return res


# ---------------------------------------------------------- profiling mode
COPY_BYTES = 256 << 20


def profile_run(name: str, steps: int) -> dict:
    """Workload for rocprofv3: ``steps`` x (cache flush, forward, backward) of one
    operator at its BASELINE configuration, then ``steps`` plain copies of
    COPY_BYTES (a torch elementwise kernel reading and writing COPY_BYTES each),
    whose FETCH_SIZE/WRITE_SIZE readings calibrate the counters for the op's
    kernels."""
    import torch

    from evograd_amd import decls, pair_module
    from evograd_amd.bind import backward_inactive_kwargs, lookup_pair
    from evograd_amd.harness import CacheFlusher
    from evograd_amd.inputs import make_case_inputs

    base, label = split_name(name)
    op = decls.get_op(base)
    mod = pair_module(base)
    w = bench_workload(op, label)
    inputs = make_case_inputs(op, w, "cuda")
    f, b = lookup_pair(op, mod)
    args = [inputs.get(a.name, getattr(a, "default", None)) for a in op.args]
    kw = backward_inactive_kwargs(op, b, inputs)
    dy = inputs[op.upstream_grad_name]
    flush = CacheFlusher("cuda")
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    times = {"fwd": [], "bwd": [], "copy": []}
    for _ in range(steps):
        flush()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        _, saved = f(*args)
        e[1].record()
        b(dy, saved, **kw)
        e[2].record()
        torch.cuda.synchronize()
        times["fwd"].append(e[0].elapsed_time(e[1]) * 1e3)
        times["bwd"].append(e[1].elapsed_time(e[2]) * 1e3)
    for _ in range(steps):
        flush()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        e[0].record()
        torch.mul(src, 1.0, out=dst)
        e[1].record()
        torch.cuda.synchronize()
        times["copy"].append(e[0].elapsed_time(e[1]) * 1e3)
    return {"profile": name, "config": {"dims": w.dims, "dtype": w.dtype},
            "copy_bytes_each_way": COPY_BYTES,
            **{f"{k}_us_median": statistics.median(v) for k, v in times.items()}}


def load_traffic(kernel_key: str):
    """HBM bytes per launch of a kernel, measured by rocprofv3 FETCH_SIZE and
    WRITE_SIZE runs and recorded under profiles/ (None when not measured)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as fh:
            entry = json.load(fh).get(kernel_key)
    except (OSError, ValueError):
        return None
    return entry


# --------------------------------------------------------------------- main
def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ops", default=",".join(ALL_OPS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the token sweeps of the memory-bound operators")
    ap.add_argument("--no-eager", action="store_true",
                    help="skip the eager torch baseline on the GPU")
    ap.add_argument("--profile", metavar="OP",
                    help="rocprofv3 workload: STEPS x (flush, fwd, bwd) of OP plus copy calibration; "
                         "'sustained' runs the MFMA probe and the HBM copy STEPS times")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: every operator's work shards by rows, tokens or "
              "heads with no exchange or one 16 KB all-reduce of the norm parameter gradients, "
              "and no multi-GPU run is part of this build.",
              file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    from evograd_amd import _lib
    from evograd_amd.harness import CacheFlusher

    _lib.load()
    torch.cuda.set_device(0)
    if args.profile == "sustained":
        print(json.dumps(sustained_rates(args.steps)), flush=True)
        return 0
    if args.profile:
        print(json.dumps(profile_run(args.profile, args.steps)), flush=True)
        return 0
    flush = CacheFlusher("cuda")
    ops = [o for o in args.ops.split(",") if o]
    if HEADLINE not in ops:
        ops.insert(0, HEADLINE)
    results = {}
    torch.cuda.synchronize()
    for name in ops:
        log(f"gpu {name} ...")
        try:
            results[name] = gpu_op(name, args.steps, args.warmup, flush)
        except Exception as e:  # recorded, as the reference's harness does
            results[name] = {"error": f"{type(e).__name__}: {e}"}
            if name == HEADLINE:
                raise
        log(f"gpu {name}: " + json.dumps({k: v for k, v in results[name].items()
                                          if k in ("fwd_us", "bwd_us", "full_us", "error")}))
    torch.cuda.synchronize()
    sweeps = {}
    if not args.no_sweep:
        for name in SWEEP_OPS:
            if name.split("@")[0] not in [o.split("@")[0] for o in ops]:
                continue
            log(f"sweep {name} ...")
            try:
                sweeps[name] = sweep_op(name, SWEEP_OPS[name], max(5, args.steps // 2),
                                        min(args.warmup, 3), flush)
            except Exception as e:
                sweeps[name] = {"error": f"{type(e).__name__}: {e}"}
            log(f"sweep {name}: " + json.dumps({k: v.get("hbm_frac_full") if isinstance(v, dict)
                                                else v for k, v in sweeps[name].items()}))

    if not args.no_eager:
        for name in ops:
            if name not in EAGER_OPS or "full_us" not in results.get(name, {}):
                continue
            log(f"gpu eager {name} ...")
            try:
                eg = gpu_eager(name, max(5, args.steps // 2), 2, flush)
                results[name]["gpu_eager_full_us"] = eg["full_us"]
                results[name]["speedup_vs_gpu_eager"] = round(eg["full_us"] / results[name]["full_us"], 3)
                if "note" in eg:
                    results[name]["gpu_eager_note"] = eg["note"]
            except Exception as e:
                results[name]["gpu_eager_error"] = f"{type(e).__name__}: {e}"
            log(f"gpu eager {name}: " + json.dumps({k: v for k, v in results[name].items()
                                                     if k.startswith(("gpu_eager", "speedup_vs_gpu"))}))
    log("sustained rates ...")
    try:
        sustained = sustained_rates()
    except Exception as e:
        sustained = {"error": f"{type(e).__name__}: {e}"}
    log("sustained rates: " + json.dumps({k: v for k, v in sustained.items() if k != "how"}))
    if "mfma_bf16_tflops" in sustained:
        for r in results.values():
            if "mfma_frac_full" in r:
                r["mfma_frac_full_of_sustained"] = round(
                    r["mfma_frac_full"] * BF16_PEAK_TFLOPS / sustained["mfma_bf16_tflops"], 4)

    cpu = {}
    if not args.no_cpu:
        for name in ops:
            log(f"cpu {name} ...")
            try:
                cpu[name] = cpu_baseline(name)
            except Exception as e:
                cpu[name] = {"error": f"{type(e).__name__}: {e}"}
            if "value" in results.get(name, {}) or "full_us" in results.get(name, {}):
                if "value" in cpu[name]:
                    results[name]["cpu_full_us"] = cpu[name]["value"]
                    results[name]["speedup_vs_cpu"] = cpu[name]["value"] / results[name]["full_us"]

    head = results[HEADLINE]
    w = head["config"]
    dims = w["dims"]
    # Dominant kernel of the headline step: the RMSNorm backward ring kernel
    # (norm_bwd_ring: reads dy, x, rstd, weight; writes dx and the partial rows),
    # its duration from events the dispatch records.
    dk = head["dominant_kernel"]
    achieved = dk["achieved_gbs"]
    line = {
        "metric": METRIC,
        "value": round(head["full_us"], 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["full_us"] / 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"rmsnorm fwd+bwd bf16 x[{dims['rows']},{dims['hidden']}] eps=1e-6 "
                        "(BASELINE configs[1])",
            "rows": dims["rows"], "hidden": dims["hidden"],
            "parallelism": "single-gpu",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dk["name"],
            "kernel_us": round(dk["us"], 2),
            "algorithmic_bytes": dk["bytes"],
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
        },
        "cpu_baseline": ({k: v for k, v in cpu[HEADLINE].items() if k != "what"}
                         if HEADLINE in cpu and "value" in cpu[HEADLINE] else None),
        "cpu_model": cpu_model(),
        "sustained": sustained,
        "ops": results,
        "sweeps": sweeps,
    }
    traffic = load_traffic("norm_bwd_ring")
    if traffic is not None:
        line["roofline"]["traffic"] = traffic.get("hbm_bytes_per_launch")
        line["roofline"]["traffic_source"] = "profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated)"
    if "hbm_copy_gbs" in sustained:
        line["roofline"]["frac_of_sustained_copy"] = round(achieved / sustained["hbm_copy_gbs"], 4)
    if line["cpu_baseline"] is not None:
        line["cpu_baseline"]["value"] = round(line["cpu_baseline"]["value"], 1)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
