"""Loader of the golden fixtures in tests/golden/ (written by make_golden.py)."""

import os

import numpy as np
import torch

from evograd_amd import decls

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
OPS = ("softmax", "rmsnorm", "layernorm", "swiglu", "rope", "fused_add_rms_norm",
       "causal_attention", "causal_attention_gqa", "llama3_attention", "cross_entropy",
       "fused_linear_cross_entropy", "llama3_decoder_layer")
TABLE_ARGS = {"rope": ("cos", "sin"), "llama3_attention": ("cos", "sin"),
              "llama3_decoder_layer": ("cos", "sin")}


def load(op_name: str) -> dict:
    with np.load(os.path.join(GOLDEN, f"{op_name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def case_inputs(op_name: str, dtype: torch.dtype, device: str) -> tuple:
    """(inputs keyed by declared names + upstream grad, expected output, expected
    gradients keyed by gradient name); float inputs in ``dtype``, integer ones as
    int64, rotary tables kept fp32."""
    op = decls.get_op(op_name)
    g = load(op_name)
    inputs = {}
    for arg in op.args:
        key = f"in_{arg.name}"
        if key in g:
            a = g[key]
            if a.dtype.kind in "iu":
                inputs[arg.name] = torch.from_numpy(a).to(device)
            else:
                dt = torch.float32 if arg.name in TABLE_ARGS.get(op_name, ()) else dtype
                inputs[arg.name] = torch.from_numpy(a).to(device=device, dtype=dt)
        elif f"scalar_{arg.name}" in g:
            inputs[arg.name] = float(g[f"scalar_{arg.name}"])
    inputs[op.upstream_grad_name] = torch.from_numpy(g["dy"]).to(device=device, dtype=dtype)
    expected = torch.from_numpy(g["out"])
    grads = {name: torch.from_numpy(g[f"grad_{name}"]) for name in op.grad_names()}
    return inputs, expected, grads


def assert_close(name, actual, expected, rtol, atol_frac):
    """|a - e| <= rtol |e| + atol_frac * max|e| elementwise."""
    a = actual.detach().double().cpu()
    e = expected.double()
    assert a.shape == e.shape, (name, tuple(a.shape), tuple(e.shape))
    scale = float(e.abs().max()) if e.numel() else 0.0
    err = (a - e).abs()
    bound = rtol * e.abs() + atol_frac * scale
    worst = float((err - bound).max()) if e.numel() else 0.0
    assert worst <= 0, f"{name}: max err {float(err.max()):.3g} exceeds the bound by {worst:.3g}"
