"""Deterministic seeded synthetic inputs per declared workload.

Restates src/evograd/opdecl/inputs.py:40-75 and the declarations' ``make_inputs``
recipes (seeds and distributions), so a case means the same tensors here as in
the reference's harness on the same device type.
"""

from __future__ import annotations

import torch

from .opdecl import Active, OpDecl, Workload, bind_shape

DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
          "float64": torch.float64}

# Llama-3's rotary base (src/evograd/opdecl/models.py:259-261); the benchmark RoPE
# configuration (label "baseline") overrides it with theta=10000 through the workload's ``extra``.
LLAMA3_ROPE_THETA = 500000.0


def resolve_dtype(name: str) -> torch.dtype:
    try:
        return DTYPES[name]
    except KeyError:
        raise ValueError(f"unsupported dtype {name!r}") from None


def case_seed(workload: Workload) -> int:
    """Generic per-case seed (inputs.py:40-49)."""
    seed = 0
    for name in sorted(workload.dims):
        seed = seed * 131 + int(workload.dims[name])
    return seed * 131 + sum(map(ord, workload.dtype))


def make_softmax_inputs(op, workload, device="cuda"):
    """softmax/__init__.py:44-51: seed rows*100003+cols, x then dy ~ N(0,1)."""
    rows, cols = workload.dims["rows"], workload.dims["cols"]
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(rows * 100003 + cols)
    x = torch.randn((rows, cols), device=device, dtype=dt)
    dy = torch.randn((rows, cols), device=device, dtype=dt)
    return {"x": x, "dy": dy}


def make_rmsnorm_inputs(op, workload, device="cuda"):
    """rmsnorm/__init__.py:20-32: seed rows*100000+hidden; x; weight = 1 + 0.1 N(0,1)
    drawn in fp32 then cast; dy. eps 1e-5 unless the workload says otherwise."""
    rows, hidden = workload.dims["rows"], workload.dims["hidden"]
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(rows * 100000 + hidden)
    x = torch.randn((rows, hidden), device=device, dtype=dt)
    weight = (1.0 + 0.1 * torch.randn((hidden,), device=device, dtype=torch.float32)).to(dt)
    dy = torch.randn((rows, hidden), device=device, dtype=dt)
    return {"x": x, "weight": weight, "eps": float(workload.extra.get("eps", 1e-5)), "dy": dy}


def make_fused_add_rms_norm_inputs(op, workload, device="cuda"):
    """fused_add_rms_norm/__init__.py:55-64: seed rows*100003+cols; x, r, weight, dout
    ~ N(0,1) in that order; eps 1e-6."""
    rows, cols = workload.dims["rows"], workload.dims["cols"]
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(rows * 100003 + cols)
    x = torch.randn((rows, cols), device=device, dtype=dt)
    r = torch.randn((rows, cols), device=device, dtype=dt)
    weight = torch.randn((cols,), device=device, dtype=dt)
    dout = torch.randn((rows, cols), device=device, dtype=dt)
    return {"x": x, "r": r, "weight": weight, "eps": float(workload.extra.get("eps", 1e-6)),
            "dout": dout}


def make_layernorm_inputs(op, workload, device="cuda"):
    """layernorm/__init__.py:16-24: seed rows*100000+hidden; x, weight, bias, dy ~ N(0,1)."""
    rows, hidden = workload.dims["rows"], workload.dims["hidden"]
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(rows * 100000 + hidden)
    x = torch.randn((rows, hidden), device=device, dtype=dt)
    weight = torch.randn((hidden,), device=device, dtype=dt)
    bias = torch.randn((hidden,), device=device, dtype=dt)
    dy = torch.randn((rows, hidden), device=device, dtype=dt)
    return {"x": x, "weight": weight, "bias": bias,
            "eps": float(workload.extra.get("eps", 1e-5)), "dy": dy}


def make_swiglu_inputs(op, workload, device="cuda"):
    """swiglu/__init__.py:44-52: seed rows*100003+cols; a, b, dc ~ N(0,1)."""
    rows, cols = workload.dims["rows"], workload.dims["cols"]
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(rows * 100003 + cols)
    a = torch.randn((rows, cols), device=device, dtype=dt)
    b = torch.randn((rows, cols), device=device, dtype=dt)
    dc = torch.randn((rows, cols), device=device, dtype=dt)
    return {"a": a, "b": b, "dc": dc}


def rope_tables(tokens: int, head_dim: int, theta: float, dtype, device):
    """cos/sin [tokens, head_dim] with duplicated halves (rope/__init__.py:47-59):
    angle[t, i] = t * theta^(-2i/head_dim), i < head_dim/2."""
    positions = torch.arange(tokens, device=device, dtype=torch.float32)[:, None]
    inv_freq = theta ** (
        -torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim
    )
    freqs = positions * inv_freq[None, :]
    angles = torch.cat((freqs, freqs), dim=-1)
    return angles.cos().to(dtype), angles.sin().to(dtype)


def make_rope_inputs(op, workload, device="cuda"):
    """rope/__init__.py:30-62: seed T*100003 + heads*1009 + head_dim; x = 0.5 N(0,1);
    tables at Llama-3's theta cast to x's dtype; dy = 0.5 N(0,1). A workload's
    ``extra`` may set theta, table_dtype and x_scale (the benchmark case uses
    theta 10000, fp32 tables and unit-variance x)."""
    d = workload.dims
    B, H, T, D = d["B"], d["n_heads"], d["T"], d["head_dim"]
    if D % 2:
        raise ValueError(f"rope needs an even head_dim, got {D}")
    dt = resolve_dtype(workload.dtype)
    scale = float(workload.extra.get("x_scale", 0.5 if workload.label != "baseline" else 1.0))
    torch.manual_seed(T * 100003 + H * 1009 + D)
    x = torch.randn((B, H, T, D), device=device, dtype=dt) * scale
    theta = float(workload.extra.get("theta", LLAMA3_ROPE_THETA))
    tdt = resolve_dtype(workload.extra.get("table_dtype", workload.dtype))
    cos, sin = rope_tables(T, D, theta, tdt, device)
    dy = torch.randn((B, H, T, D), device=device, dtype=dt) * scale
    return {"x": x, "cos": cos, "sin": sin, "dy": dy}


def make_attention_inputs(op, workload, device="cuda"):
    """Generic seed (inputs.py:40-49); q, k, v, do ~ N(0,1) as the benchmark
    attention configuration specifies."""
    d = workload.dims
    shape = (d["B"], d["H"], d["S"], d["D"])
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(case_seed(workload))
    q = torch.randn(shape, device=device, dtype=dt)
    k = torch.randn(shape, device=device, dtype=dt)
    v = torch.randn(shape, device=device, dtype=dt)
    do = torch.randn(shape, device=device, dtype=dt)
    return {"q": q, "k": k, "v": v, "do": do}


def make_attention_gqa_inputs(op, workload, device="cuda"):
    """Generic seed (inputs.py:40-49); q, do [B, H, S, D] and k, v [B, KVH, S, D]
    ~ N(0,1), drawn in the order q, k, v, do."""
    d = workload.dims
    qs = (d["B"], d["H"], d["S"], d["D"])
    ks = (d["B"], d["KVH"], d["S"], d["D"])
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(case_seed(workload))
    q = torch.randn(qs, device=device, dtype=dt)
    k = torch.randn(ks, device=device, dtype=dt)
    v = torch.randn(ks, device=device, dtype=dt)
    do = torch.randn(qs, device=device, dtype=dt)
    return {"q": q, "k": k, "v": v, "do": do}


def make_llama3_attention_inputs(op, workload, device="cuda"):
    """Generic seed (inputs.py:40-49); q [B, H, S, D], k, v [B, KVH, S, D], do
    [B, H, S, D] ~ N(0,1) drawn in that order; cos/sin [S, D] fp32 tables at
    Llama-3's theta (``extra`` may set theta and table_dtype), the decoder layer's
    tables (src/evograd/ops/level3/llama3_decoder_layer/__init__.py:106-123)."""
    d = workload.dims
    qs = (d["B"], d["H"], d["S"], d["D"])
    ks = (d["B"], d["KVH"], d["S"], d["D"])
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(case_seed(workload))
    q = torch.randn(qs, device=device, dtype=dt)
    k = torch.randn(ks, device=device, dtype=dt)
    v = torch.randn(ks, device=device, dtype=dt)
    do = torch.randn(qs, device=device, dtype=dt)
    theta = float(workload.extra.get("theta", LLAMA3_ROPE_THETA))
    tdt = resolve_dtype(workload.extra.get("table_dtype", "float32"))
    cos, sin = rope_tables(d["S"], d["D"], theta, tdt, device)
    return {"q": q, "k": k, "v": v, "cos": cos, "sin": sin, "do": do}


def make_cross_entropy_inputs(op, workload, device="cuda"):
    """cross_entropy/__init__.py:48-56: seed rows*100003+cols; logits ~ N(0,1), target
    uniform in [0, cols) (int64), dloss = U[0,1) + 0.5 (0-dim, logits dtype), drawn in
    that order. ``extra["ignore_every"] = k`` then sets every k-th target (rows 0, k,
    2k, ...) to the ignore index -100."""
    rows, cols = workload.dims["rows"], workload.dims["cols"]
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(rows * 100003 + cols)
    logits = torch.randn((rows, cols), device=device, dtype=dt)
    target = torch.randint(0, cols, (rows,), device=device, dtype=torch.int64)
    dloss = torch.rand((), device=device, dtype=dt) + 0.5
    every = int(workload.extra.get("ignore_every", 0))
    if every:
        target[::every] = -100
    return {"logits": logits, "target": target, "dloss": dloss}


def make_flce_inputs(op, workload, device="cuda"):
    """fused_linear_cross_entropy/__init__.py:34-55: seed rows*100003 + hidden*1009 +
    vocab; x = 0.5 N(0,1); weight = N(0,1) / sqrt(hidden) drawn in fp32 then cast;
    target uniform in [0, vocab); dloss = 1 (0-dim, input dtype). ``extra
    ["ignore_every"] = k`` then sets targets 0, k, 2k, ... to -100."""
    rows, hidden, vocab = workload.dims["rows"], workload.dims["hidden"], workload.dims["vocab"]
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(rows * 100003 + hidden * 1009 + vocab)
    x = torch.randn((rows, hidden), device=device, dtype=dt) * 0.5
    weight = (torch.randn((vocab, hidden), device=device, dtype=torch.float32)
              * hidden ** -0.5).to(dt)
    target = torch.randint(0, vocab, (rows,), device=device, dtype=torch.int64)
    dloss = torch.ones((), device=device, dtype=dt)
    every = int(workload.extra.get("ignore_every", 0))
    if every:
        target[::every] = -100
    return {"x": x, "weight": weight, "target": target, "dloss": dloss}


def make_llama3_decoder_layer_inputs(op, workload, device="cuda"):
    """llama3_decoder_layer/__init__.py:68-133: seed T*100003 + hidden*1009 + head_dim;
    drawn in this order: x = 0.5 N(0,1) [B, T, hidden]; input_norm_weight = 1 + 0.1
    N(0,1) (fp32 draw, cast); q/k/v/o weights N(0,1) * in^-0.5 (fp32 draw, cast,
    [out, in]); post_norm_weight; gate, up, down weights; then dout = 0.5 N(0,1) *
    (B*T)^-0.5. cos/sin [T, head_dim] at Llama-3's theta in x's dtype; eps 1e-5.
    The shape checks of :73-86 are kept (q_out, kv_out multiples of head_dim, whole
    GQA groups, q_out == hidden)."""
    d = workload.dims
    batch, tokens, hidden = d["B"], d["T"], d["hidden"]
    head_dim, q_out, kv_out, inter = d["head_dim"], d["q_out"], d["kv_out"], d["intermediate"]
    if q_out % head_dim or kv_out % head_dim:
        raise ValueError("q_out and kv_out must be whole multiples of head_dim")
    n_heads, n_kv = q_out // head_dim, kv_out // head_dim
    if n_heads % n_kv:
        raise ValueError(f"GQA needs n_heads divisible by n_kv_heads, got {n_heads} and {n_kv}")
    if q_out != hidden:
        raise ValueError("Llama-3 ties n_heads*head_dim to hidden")
    dt = resolve_dtype(workload.dtype)
    torch.manual_seed(tokens * 100003 + hidden * 1009 + head_dim)

    def weight(out_features, in_features):
        return (torch.randn((out_features, in_features), device=device, dtype=torch.float32)
                * in_features ** -0.5).to(dt)

    def gain(width):
        return (1.0 + 0.1 * torch.randn((width,), device=device, dtype=torch.float32)).to(dt)

    out = {"x": torch.randn((batch, tokens, hidden), device=device, dtype=dt) * 0.5}
    out["input_norm_weight"] = gain(hidden)
    out["q_weight"] = weight(q_out, hidden)
    out["k_weight"] = weight(kv_out, hidden)
    out["v_weight"] = weight(kv_out, hidden)
    out["o_weight"] = weight(hidden, q_out)
    out["post_norm_weight"] = gain(hidden)
    out["gate_weight"] = weight(inter, hidden)
    out["up_weight"] = weight(inter, hidden)
    out["down_weight"] = weight(hidden, inter)
    theta = float(workload.extra.get("theta", LLAMA3_ROPE_THETA))
    out["cos"], out["sin"] = rope_tables(tokens, head_dim, theta, dt, device)
    out["eps"] = 1e-5
    out["dout"] = (torch.randn((batch, tokens, hidden), device=device, dtype=dt) * 0.5
                   * (batch * tokens) ** -0.5)
    return out


RECIPES = {
    "make_softmax_inputs": make_softmax_inputs,
    "make_rmsnorm_inputs": make_rmsnorm_inputs,
    "make_layernorm_inputs": make_layernorm_inputs,
    "make_fused_add_rms_norm_inputs": make_fused_add_rms_norm_inputs,
    "make_swiglu_inputs": make_swiglu_inputs,
    "make_rope_inputs": make_rope_inputs,
    "make_attention_inputs": make_attention_inputs,
    "make_attention_gqa_inputs": make_attention_gqa_inputs,
    "make_llama3_attention_inputs": make_llama3_attention_inputs,
    "make_cross_entropy_inputs": make_cross_entropy_inputs,
    "make_flce_inputs": make_flce_inputs,
    "make_llama3_decoder_layer_inputs": make_llama3_decoder_layer_inputs,
}


def make_case_inputs(op: OpDecl, workload: Workload, device: str = "cuda") -> dict:
    """All primals plus the upstream gradient keyed by declared names (inputs.py:52-75)."""
    if op.make_inputs is not None:
        _, _, fn = op.make_inputs.partition(":")
        return RECIPES[fn](op, workload, device)
    torch.manual_seed(case_seed(workload))
    values: dict = {}
    dt = resolve_dtype(workload.dtype)
    for arg in op.args:
        if isinstance(arg, Active):
            values[arg.name] = torch.randn(bind_shape(arg.shape, workload.dims), device=device,
                                           dtype=dt) * 0.5
        elif arg.is_tensor:
            values[arg.name] = torch.zeros(bind_shape(arg.shape, workload.dims), device=device,
                                           dtype=dt)
        else:
            values[arg.name] = arg.default
    values[op.upstream_grad_name] = torch.randn(
        bind_shape(op.output.shape, workload.dims), device=device, dtype=dt) * 0.5
    return values
