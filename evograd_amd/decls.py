"""Declarations of the autograd-pair operators this library implements.

Argument names, activity, output and gradient names follow the reference's
declarations exactly, so a candidate module written against them is the same
drop-in the reference's harness looks up:

* softmax    src/evograd/ops/level1/softmax/__init__.py:69-92
* rmsnorm    src/evograd/ops/level1/rmsnorm/__init__.py:72-130
* layernorm  src/evograd/ops/level1/layernorm/__init__.py:124-171
* swiglu     src/evograd/ops/level1/swiglu/__init__.py:61-97
* rope       src/evograd/ops/level1/rope/__init__.py:98-162
* fused_add_rms_norm  src/evograd/ops/level2/fused_add_rms_norm/__init__.py:76-122
* cross_entropy  src/evograd/ops/level1/cross_entropy/__init__.py:76-111
* fused_linear_cross_entropy  src/evograd/ops/level2/fused_linear_cross_entropy/__init__.py:91-152
* llama3_decoder_layer  src/evograd/ops/level3/llama3_decoder_layer/__init__.py:136-235
* causal_attention: the reference has no standalone declaration; its semantics
  are F.scaled_dot_product_attention(q, k, v, is_causal=True) inside
  src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:101-108. It is
  declared here the way an external ``--declaration path.py:op`` would be
  (src/evograd/opdecl/verify_cli.py:35-38).

Differences from the reference declarations, all deliberate:

* Tolerances are the stricter gate of this build: fp32 (1e-5, 1e-5),
  fp16 (1e-2, 1e-2), bf16 (2e-2, 2e-2), flat for every output and gradient (the
  reference uses fp32 2e-5, fp16 5e-2, bf16 8e-2, src/evograd/ops/_common.py:13-17,
  and widens bf16 parameter gradients by sqrt(rows/8)). The one exception is the
  decoder layer, which keeps the reference's own block-level gate (below).
* ``reference_dtype="float32"``: the oracle runs reduced-precision cases in fp32
  and casts back (the promotion of src/evograd/opdecl/oracle.py:70-110), so a
  comparison measures the kernel's error, not the oracle's own bf16 rounding.
* Each declaration also lists the benchmark configuration(s) of this build as
  ``benchmark`` workloads (label "baseline").

``forward``/``runtime_forward`` are "module:function" strings naming the
CPU-checkable restatement in the repository's ``oracle`` package, which only
tests and the benchmark's CPU baseline import; ``make_inputs`` names the seeded
input recipe in ``evograd_amd.inputs``.
"""

from __future__ import annotations

from .opdecl import Active, Inactive, OpDecl, Workload, declare_op

TOLERANCES = {
    "float32": (1e-5, 1e-5),
    "float16": (1e-2, 1e-2),
    "bfloat16": (2e-2, 2e-2),
}


# Shape regimes of the reference declarations: the row (token) count splits small
# from large shapes at Llama-3's 4096 tokens (2048 for vocabulary-wide rows),
# src/evograd/opdecl/models.py:306-307.
LLAMA_REGIME_SPLIT = 4096.0
LLAMA_VOCAB_REGIME_SPLIT = 2048.0


def _rows_feature(workload) -> float:
    return float(workload.dims["rows"])


def _tokens_feature(workload) -> float:
    return float(workload.dims["T"])


def _seq_feature(workload) -> float:
    return float(workload.dims["S"])


def _w2(shapes, dtypes, row="rows", col="cols", label=""):
    return tuple(
        Workload(dims={row: r, col: c}, dtype=dt, label=label)
        for (r, c) in shapes
        for dt in dtypes
    )


# ------------------------------------------------------------------ softmax
SOFTMAX = declare_op(
    name="softmax",
    forward="oracle.forward_refs:softmax_forward_ref",
    dims=("rows", "cols"),
    args=(Active("x", "[rows, cols]"),),
    output=Active("y", "[rows, cols]"),
    forward_semantics="Numerically stable softmax over the last dimension in fp32.",
    backward_semantics="Return dx = y * (dy - sum(dy*y, dim=-1, keepdim=True)).",
    reference_dtype="float32",
    correctness=(
        _w2(((8, 512), (16, 1024)), ("float32",))
        + _w2(((32, 4096), (64, 2048)), ("float16", "bfloat16"))
        # ragged widths (scalar path), a single row and a vocabulary-wide row
        # (16-bit: row in registers as raw packs; fp32: two-read path)
        + _w2(((17, 1000), (5, 127), (1, 4096), (3, 131072)), ("float32", "bfloat16"))
        # a partly filled register row (fp16, bf16) and a row past the register
        # path (two-read path for 16-bit types)
        + _w2(((3, 100000),), ("float16", "bfloat16"))
        # the narrowest row past the one-register-row kernels: most of a thread's packs
        # lie past the row (bounded loads return zeros, LDS slots stay unwritten)
        + _w2(((2, 65600),), ("bfloat16",))
        + _w2(((2, 262144),), ("bfloat16",))
    ),
    # The fp32 [4096, 4096] benchmark case, and the reference's timed default width (bf16
    # rows of the Llama-3 vocabulary, src/evograd/ops/level1/softmax/__init__.py:31-37)
    benchmark=(_w2(((4096, 4096),), ("float32",), label="baseline")
               + _w2(((4096, 128256),), ("bfloat16",), label="vocab")),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_softmax_inputs",
    regime_feature=_rows_feature,
    regime_split=LLAMA_VOCAB_REGIME_SPLIT,
)

# ------------------------------------------------------------------ rmsnorm
RMSNORM = declare_op(
    name="rmsnorm",
    forward="oracle.forward_refs:rmsnorm_forward_ref",
    runtime_forward="oracle.forward_refs:rmsnorm_runtime_ref",
    dims=("rows", "hidden"),
    args=(
        Active("x", "[rows, hidden]"),
        Active("weight", "[hidden]"),
        Inactive("eps", default=1e-5),
    ),
    output=Active("y", "[rows, hidden]"),
    forward_semantics=(
        "rrms = rsqrt(mean(x^2, -1) + eps) in fp32; y = ((x * rrms) * weight) cast to "
        "x's dtype."
    ),
    backward_semantics=(
        "xhat = x * rrms, g = dy * weight: dx = (g - xhat * mean(g * xhat, -1)) * rrms; "
        "dweight = sum(dy * xhat, dim=0); fp32 accumulation."
    ),
    reference_dtype="float32",
    correctness=(
        Workload(dims=dict(rows=8, hidden=64), dtype="float32"),
        Workload(dims=dict(rows=17, hidden=128), dtype="float32"),
        Workload(dims=dict(rows=32, hidden=256), dtype="float16"),
        Workload(dims=dict(rows=64, hidden=512), dtype="float16"),
        Workload(dims=dict(rows=32, hidden=256), dtype="bfloat16"),
        Workload(dims=dict(rows=64, hidden=512), dtype="bfloat16"),
        Workload(dims=dict(rows=128, hidden=4096), dtype="bfloat16"),
        # coverage: single and ragged row counts, non-power-of-two widths,
        # more rows than backward workgroups, the widest Llama hidden
        Workload(dims=dict(rows=1, hidden=4096), dtype="bfloat16"),
        Workload(dims=dict(rows=17, hidden=127), dtype="float32"),
        Workload(dims=dict(rows=17, hidden=513), dtype="float16"),
        Workload(dims=dict(rows=17, hidden=1000), dtype="bfloat16"),
        Workload(dims=dict(rows=1500, hidden=768), dtype="bfloat16"),
        Workload(dims=dict(rows=1024, hidden=8192), dtype="bfloat16"),
        # rows of 512 packs (one workgroup per row in the forward) in the other dtypes
        Workload(dims=dict(rows=33, hidden=2048), dtype="float32"),
        Workload(dims=dict(rows=9, hidden=4096), dtype="float16"),
    ),
    benchmark=(
        Workload(dims=dict(rows=16384, hidden=4096), dtype="bfloat16", label="baseline",
                 extra={"eps": 1e-6}),
    ),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_rmsnorm_inputs",
    regime_feature=_rows_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# ------------------------------------------------------- fused_add_rms_norm
# Correctness: the reference's standard 2-D shapes (src/evograd/ops/_common.py:18-22)
# plus ragged/wide rows; benchmark: its Llama-3-8B residual-stream workload at the
# largest token count of the sweep (rows = 16384 tokens, cols = hidden 4096).
FUSED_ADD_RMS_NORM = declare_op(
    name="fused_add_rms_norm",
    forward="oracle.forward_refs:fused_add_rms_norm_forward_ref",
    runtime_forward="oracle.forward_refs:fused_add_rms_norm_runtime_ref",
    dims=("rows", "cols"),
    args=(
        Active("x", "[rows, cols]"),
        Active("r", "[rows, cols]"),
        Active("weight", "[cols]"),
        Inactive("eps", default=1e-6),
    ),
    output=Active("out", "[rows, cols]"),
    forward_semantics=(
        "Set s=x+r, compute rstd=rsqrt(mean(s**2,lastdim)+eps) in fp32, "
        "and return s*rstd*weight."
    ),
    backward_semantics=(
        "Return dx, dr, dweight. dx and dr are the same gradient through s; "
        "dweight reduces dout*s*rstd across rows."
    ),
    reference_dtype="float32",
    correctness=(
        _w2(((8, 64), (17, 128)), ("float32",))
        + _w2(((32, 256), (64, 512)), ("float16", "bfloat16"))
        + (
            Workload(dims=dict(rows=1, cols=4096), dtype="bfloat16"),
            Workload(dims=dict(rows=17, cols=1000), dtype="bfloat16"),
            Workload(dims=dict(rows=17, cols=127), dtype="float32"),
            Workload(dims=dict(rows=1500, cols=1024), dtype="bfloat16"),
            Workload(dims=dict(rows=300, cols=4096), dtype="bfloat16"),
            Workload(dims=dict(rows=33, cols=2048), dtype="float32"),
            Workload(dims=dict(rows=9, cols=4096), dtype="float16"),
        )
    ),
    benchmark=(
        Workload(dims=dict(rows=16384, cols=4096), dtype="bfloat16", label="llama3_8b"),
    ),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_fused_add_rms_norm_inputs",
    regime_feature=_rows_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# ---------------------------------------------------------------- layernorm
LAYERNORM = declare_op(
    name="layernorm",
    forward="oracle.forward_refs:layernorm_forward_ref",
    runtime_forward="oracle.forward_refs:layernorm_runtime_ref",
    dims=("rows", "hidden"),
    args=(
        Active("x", "[rows, hidden]"),
        Active("weight", "[hidden]"),
        Active("bias", "[hidden]"),
        Inactive("eps", default=1e-5),
    ),
    output=Active("y", "[rows, hidden]"),
    forward_semantics="Row-wise LayerNorm over the last dimension, statistics in fp32.",
    backward_semantics=(
        "Return dx, dweight, dbias from dy, saved state and eps; dtypes follow x, weight "
        "and bias."
    ),
    reference_dtype="float32",
    correctness=(
        Workload(dims=dict(rows=8, hidden=64), dtype="float32"),
        Workload(dims=dict(rows=17, hidden=128), dtype="float32"),
        Workload(dims=dict(rows=32, hidden=256), dtype="float16"),
        Workload(dims=dict(rows=64, hidden=512), dtype="float16"),
        Workload(dims=dict(rows=32, hidden=256), dtype="bfloat16"),
        Workload(dims=dict(rows=64, hidden=512), dtype="bfloat16"),
        Workload(dims=dict(rows=128, hidden=4096), dtype="bfloat16"),
        Workload(dims=dict(rows=1024, hidden=8192), dtype="bfloat16"),
        Workload(dims=dict(rows=17, hidden=1000), dtype="bfloat16"),
        Workload(dims=dict(rows=17, hidden=127), dtype="float32"),
        Workload(dims=dict(rows=1500, hidden=768), dtype="bfloat16"),
        # rows of 512 packs (one workgroup per row in the forward) in the other dtypes
        Workload(dims=dict(rows=33, hidden=2048), dtype="float32"),
        Workload(dims=dict(rows=9, hidden=4096), dtype="float16"),
    ),
    benchmark=(
        Workload(dims=dict(rows=16384, hidden=4096), dtype="bfloat16", label="baseline"),
    ),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_layernorm_inputs",
    regime_feature=_rows_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# ------------------------------------------------------------------- swiglu
SWIGLU = declare_op(
    name="swiglu",
    forward="oracle.forward_refs:swiglu_forward_ref",
    dims=("rows", "cols"),
    args=(Active("a", "[rows, cols]"), Active("b", "[rows, cols]")),
    output=Active("c", "[rows, cols]"),
    forward_semantics="Element-wise c = silu(a) * b, with SiLU evaluated in fp32.",
    backward_semantics=(
        "With s=sigmoid(a): db = dc*(a*s), da = dc*b*((a*s)*(1-s)+s). Preserve input dtypes."
    ),
    reference_dtype="float32",
    correctness=(
        _w2(((8, 64), (17, 128)), ("float32",))
        + _w2(((32, 256), (64, 512)), ("float16", "bfloat16"))
        + _w2(((17, 255), (17, 1001), (1, 512)), ("float32", "bfloat16"))
    ),
    benchmark=_w2(((16384, 14336),), ("bfloat16",), label="baseline"),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_swiglu_inputs",
    backward_may_overwrite=("a", "b"),
    regime_feature=_rows_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# --------------------------------------------------------------------- rope
ROPE = declare_op(
    name="rope",
    forward="oracle.forward_refs:rope_forward_ref",
    dims=("B", "n_heads", "T", "head_dim"),
    args=(
        Active("x", "[B, n_heads, T, head_dim]"),
        Inactive("cos", "[T, head_dim]", note="rotary cosine table, duplicated halves"),
        Inactive("sin", "[T, head_dim]", note="rotary sine table, same layout as cos"),
    ),
    output=Active("y", "[B, n_heads, T, head_dim]"),
    forward_semantics=(
        "Half-rotated (GPT-NeoX / Llama) RoPE: y = [x1, x2]*[cos, cos] + [-x2, x1]*[sin, sin] "
        "in fp32, cast back to x's dtype."
    ),
    backward_semantics="dx = [dy1, dy2]*[cos, cos] + [dy2, -dy1]*[sin, sin].",
    reference_dtype="float32",
    correctness=tuple(
        Workload(dims=dict(B=b, n_heads=h, T=t, head_dim=d), dtype=dt)
        for b, h, t, d in ((1, 4, 16, 64), (2, 8, 128, 128), (1, 32, 129, 128), (1, 3, 7, 10),
                           (2, 6, 33, 128))  # 6 heads: a full and a partial group of four
        for dt in ("float32", "float16", "bfloat16")
    ),
    benchmark=(
        # the q half of the joint q/k configuration; the k half has n_heads=8
        Workload(dims=dict(B=8, n_heads=32, T=4096, head_dim=128), dtype="bfloat16",
                 label="baseline", extra={"theta": 10000.0, "table_dtype": "float32",
                                          "k_heads": 8}),
    ),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_rope_inputs",
    memory_inputs=("x",),
    regime_feature=_tokens_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# --------------------------------------------------------- causal attention
CAUSAL_ATTENTION = declare_op(
    name="causal_attention",
    forward="oracle.forward_refs:causal_attention_forward_ref",
    runtime_forward="oracle.forward_refs:causal_attention_runtime_ref",
    dims=("B", "H", "S", "D"),
    args=(
        Active("q", "[B, H, S, D]"),
        Active("k", "[B, H, S, D]"),
        Active("v", "[B, H, S, D]"),
    ),
    output=Active("o", "[B, H, S, D]"),
    forward_semantics=(
        "o = softmax(q @ k^T / sqrt(D) + causal mask) @ v, the semantics of "
        "F.scaled_dot_product_attention(q, k, v, is_causal=True); fp32 accumulation."
    ),
    backward_semantics="Return dq, dk, dv; P is recomputed from the saved logsumexp.",
    reference_dtype="float32",
    correctness=tuple(
        Workload(dims=dict(B=b, H=h, S=s, D=d), dtype=dt)
        for b, h, s, d in (
            (1, 1, 1, 128),
            (1, 2, 64, 64),
            (2, 4, 128, 128),
            (1, 2, 129, 128),
            (1, 3, 200, 64),
            (1, 4, 1024, 128),
        )
        for dt in ("bfloat16", "float16")
    ) + (
        # the generic kernels: fp32, and head sizes off the MFMA path (the decoder
        # layer's correctness gate runs head_dim 32 and 16 in fp32 and bf16)
        Workload(dims=dict(B=1, H=2, S=64, D=64), dtype="float32"),
        Workload(dims=dict(B=1, H=2, S=129, D=128), dtype="float32"),
        Workload(dims=dict(B=1, H=2, S=100, D=32), dtype="float32"),
        Workload(dims=dict(B=2, H=3, S=77, D=16), dtype="float32"),
        Workload(dims=dict(B=1, H=2, S=100, D=32), dtype="bfloat16"),
        Workload(dims=dict(B=2, H=3, S=77, D=16), dtype="bfloat16"),
        Workload(dims=dict(B=1, H=2, S=70, D=48), dtype="float16"),
    ),
    benchmark=(
        Workload(dims=dict(B=4, H=32, S=4096, D=128), dtype="bfloat16", label="baseline"),
    ),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_attention_inputs",
    regime_feature=_seq_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# ----------------------------------------------- grouped-query causal attention
# The attention of src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:
# 101-107 as the layer runs it: n_kv_heads < n_heads, k and v repeated over each
# query group. Benchmark: the MHA benchmark's batch and sequence with
# Llama-3-8B's 32 query and 8 kv heads (src/evograd/opdecl/models.py:250-262).
CAUSAL_ATTENTION_GQA = declare_op(
    name="causal_attention_gqa",
    forward="oracle.forward_refs:causal_attention_gqa_forward_ref",
    runtime_forward="oracle.forward_refs:causal_attention_gqa_runtime_ref",
    dims=("B", "H", "KVH", "S", "D"),
    args=(
        Active("q", "[B, H, S, D]"),
        Active("k", "[B, KVH, S, D]"),
        Active("v", "[B, KVH, S, D]"),
    ),
    output=Active("o", "[B, H, S, D]"),
    forward_semantics=(
        "k and v repeated over each group of H/KVH query heads (repeat_interleave on "
        "the head axis), then o = softmax(q @ k^T / sqrt(D) + causal mask) @ v."
    ),
    backward_semantics=(
        "Return dq, dk, dv; dk and dv are summed over the query heads sharing each kv "
        "head; P is recomputed from the saved logsumexp."
    ),
    reference_dtype="float32",
    correctness=tuple(
        Workload(dims=dict(B=b, H=h, KVH=kv, S=s, D=d), dtype=dt)
        for b, h, kv, s, d in (
            (1, 4, 1, 64, 128),
            (2, 8, 2, 129, 128),
            (1, 4, 2, 200, 64),
            (1, 2, 2, 100, 128),
            (1, 32, 8, 512, 128),
        )
        for dt in ("bfloat16", "float16")
    ) + (
        Workload(dims=dict(B=1, H=4, KVH=1, S=32, D=32), dtype="float32"),
        Workload(dims=dict(B=2, H=4, KVH=1, S=17, D=16), dtype="float32"),
        Workload(dims=dict(B=1, H=4, KVH=2, S=100, D=64), dtype="float32"),
        Workload(dims=dict(B=1, H=4, KVH=1, S=32, D=32), dtype="bfloat16"),
        Workload(dims=dict(B=2, H=4, KVH=1, S=17, D=16), dtype="bfloat16"),
    ),
    benchmark=(
        Workload(dims=dict(B=4, H=32, KVH=8, S=4096, D=128), dtype="bfloat16",
                 label="llama3_8b"),
    ),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_attention_gqa_inputs",
    regime_feature=_seq_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# ------------------------------ RoPE(q, k) -> grouped causal attention (one pair)
# The attention half of the Llama-3 decoder layer,
# src/evograd/ops/level3/llama3_decoder_layer/forward_ref.py:93-107, as one
# autograd pair. Block-level saved-state choice (the layer's own note,
# llama3_decoder_layer/__init__.py:190-199, invites it): the pair saves the
# pre-rotation q and k (inputs, no new storage), v, o and lse, plus the tables,
# and rotates q and k again in the backward; saving the rotated q and k instead
# would add B*(H + KVH)*S*D elements of new storage to skip one rotation pass.
LLAMA3_ATTENTION = declare_op(
    name="llama3_attention",
    forward="oracle.forward_refs:llama3_attention_forward_ref",
    runtime_forward="oracle.forward_refs:llama3_attention_runtime_ref",
    dims=("B", "H", "KVH", "S", "D"),
    args=(
        Active("q", "[B, H, S, D]", note="queries before the rotation"),
        Active("k", "[B, KVH, S, D]", note="keys before the rotation"),
        Active("v", "[B, KVH, S, D]"),
        Inactive("cos", "[S, D]", note="rotary cosine table, duplicated halves"),
        Inactive("sin", "[S, D]", note="rotary sine table, same layout as cos"),
    ),
    output=Active("o", "[B, H, S, D]"),
    forward_semantics=(
        "q and k rotated (half-rotated RoPE in fp32, cast back to the input dtype), k "
        "and v repeated over each group of H/KVH query heads, then o = softmax(q_r "
        "k_r^T / sqrt(D) + causal mask) v."
    ),
    backward_semantics=(
        "Return dq, dk, dv for the pre-rotation q and k (the rotation's transpose "
        "applied to the attention gradients); dk and dv summed over each query group."
    ),
    reference_dtype="float32",
    correctness=tuple(
        Workload(dims=dict(B=b, H=h, KVH=kv, S=s, D=d), dtype=dt)
        for b, h, kv, s, d in (
            (1, 4, 1, 64, 128),
            (2, 8, 2, 129, 128),
            (1, 4, 2, 200, 64),
            (1, 2, 2, 100, 128),
            (1, 32, 8, 512, 128),
        )
        for dt in ("bfloat16", "float16")
    ),
    benchmark=(
        Workload(dims=dict(B=4, H=32, KVH=8, S=4096, D=128), dtype="bfloat16",
                 label="llama3_8b"),
    ),
    tolerances=TOLERANCES,
    make_inputs="evograd_amd.inputs:make_llama3_attention_inputs",
    memory_inputs=("q", "k", "v"),
    regime_feature=_seq_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

# ------------------------------------------------------------ cross_entropy
# src/evograd/ops/level1/cross_entropy/__init__.py:76-111. The gradient's entries
# have magnitude about dloss / (rows * cols), so a flat atol would pass anything:
# the atol of dlogits is scaled by 1 / (rows * cols) and the comparison rests on
# the relative term.
def _xent_tolerance(workload, result_name, atol, rtol):
    if result_name == "dlogits":
        atol = atol / (workload.dims["rows"] * workload.dims["cols"])
    return atol, rtol


CROSS_ENTROPY = declare_op(
    name="cross_entropy",
    forward="oracle.forward_refs:cross_entropy_forward_ref",
    dims=("rows", "cols"),
    args=(
        Active("logits", "[rows, cols]"),
        Inactive("target", "[rows]", dtype="int64"),
    ),
    output=Active("loss", "[]"),
    forward_semantics=(
        "Mean-reduced hard-label cross entropy with ignore_index=-100, no label "
        "smoothing, z-loss, or class weights; logsumexp in fp32."
    ),
    backward_semantics=(
        "dlogits = dloss * (softmax(logits) - onehot(target)) / n_valid, zero on ignored "
        "rows; target receives no gradient."
    ),
    reference_dtype="float32",
    correctness=(
        _w2(((8, 512), (16, 1024)), ("float32",))
        + _w2(((32, 4096), (64, 2048)), ("float16", "bfloat16"))
        # ragged widths (the scalar path, GPT-2's odd vocabulary), a single row, a
        # Llama-3 vocabulary row, and every third row ignored
        + _w2(((5, 127), (1, 4096), (4, 128256)), ("float32", "bfloat16"))
        + _w2(((3, 50257),), ("bfloat16",))
        + tuple(
            Workload(dims=dict(rows=r, cols=c), dtype=dt, label="ignore3",
                     extra={"ignore_every": 3})
            for r, c, dt in ((16, 1024, "float32"), (64, 2048, "bfloat16"))
        )
    ),
    # Llama-3-8B logits at the sweep's largest token count
    # (src/evograd/opdecl/models.py:84-86, :293).
    benchmark=(
        Workload(dims=dict(rows=8192, cols=128256), dtype="bfloat16", label="llama3_8b"),
    ),
    tolerances=TOLERANCES,
    tolerance_hook=_xent_tolerance,
    make_inputs="evograd_amd.inputs:make_cross_entropy_inputs",
    memory_inputs=("logits",),
    regime_feature=_rows_feature,
    regime_split=LLAMA_VOCAB_REGIME_SPLIT,
)

# ------------------------------------------------ fused_linear_cross_entropy
# src/evograd/ops/level2/fused_linear_cross_entropy/__init__.py:91-152. Like the
# reference declaration there is no reference_dtype: the forward widens x and
# weight itself and returns an fp32 loss, and the gradients come back in the
# inputs' dtypes. dx entries scale as 1/rows and dweight entries as 1/vocab
# (a softmax probability times an x entry), so their atols are scaled by those.
def _flce_tolerance(workload, result_name, atol, rtol):
    if result_name == "dx":
        atol = atol / workload.dims["rows"]
    elif result_name == "dweight":
        atol = atol / workload.dims["vocab"]
    return atol, rtol


FUSED_LINEAR_CROSS_ENTROPY = declare_op(
    name="fused_linear_cross_entropy",
    forward="oracle.forward_refs:fused_linear_cross_entropy_forward_ref",
    dims=("rows", "hidden", "vocab"),
    args=(
        Active("x", "[rows, hidden]"),
        Active("weight", "[vocab, hidden]"),
        Inactive("target", "[rows]", dtype="int64"),
    ),
    output=Active("loss", "[]"),
    forward_semantics=(
        "logits = x @ weight.T, mean hard-label cross entropy against target with "
        "ignore_index=-100; projection and logsumexp accumulated in fp32; the "
        "[rows, vocab] logits are never materialised in full."
    ),
    backward_semantics=(
        "dlogits = dloss * (softmax(logits) - onehot(target)) / n_valid; dx = dlogits @ "
        "weight, dweight = dlogits.T @ x, in the inputs' dtypes, fp32 accumulation. The "
        "same chunking the forward uses applies here: dlogits must not be materialized "
        "in full either."
    ),
    correctness=tuple(
        Workload(dims=dict(rows=r, hidden=h, vocab=v), dtype=dt)
        for r, h, v in ((8, 64, 512), (17, 128, 1000))
        for dt in ("float32", "float16", "bfloat16")
    ) + (
        # a vocabulary that is not a multiple of 4 (scalar chunk kernels) and
        # every third row ignored
        Workload(dims=dict(rows=33, hidden=64, vocab=1001), dtype="bfloat16"),
        Workload(dims=dict(rows=48, hidden=128, vocab=2048), dtype="bfloat16", label="ignore3",
                 extra={"ignore_every": 3}),
        Workload(dims=dict(rows=48, hidden=128, vocab=2048), dtype="float32", label="ignore3",
                 extra={"ignore_every": 3}),
    ),
    # Llama-3-8B lm_head at the sweep's largest token count
    # (src/evograd/opdecl/models.py:84-86, :293).
    benchmark=(
        Workload(dims=dict(rows=8192, hidden=4096, vocab=128256), dtype="bfloat16",
                 label="llama3_8b"),
    ),
    tolerances=TOLERANCES,
    tolerance_hook=_flce_tolerance,
    make_inputs="evograd_amd.inputs:make_flce_inputs",
    memory_inputs=("x", "weight"),
    regime_feature=_rows_feature,
    regime_split=LLAMA_VOCAB_REGIME_SPLIT,
)

# ------------------------------------------------------- llama3_decoder_layer
# src/evograd/ops/level3/llama3_decoder_layer/__init__.py:136-235: one Llama-3-8B
# decoder layer as one autograd pair. Its gate is the reference's own (fp32 1e-4;
# bf16 atol 5e-2 / rtol 2e-2 against the fp32 reference; atol x1.5 for the three
# widest reductions), not this build's flat per-op tolerance: at block depth the
# gradients span a dynamic range where a flat bf16 2e-2 would gate the fp32
# oracle's own rounding of ten composed operators. Correctness at the reference's
# four small workloads (:55-65); timed at its grid, B=1 and T in {1024, 2048,
# 4096} bf16 at Llama-3-8B widths (:36-44, src/evograd/opdecl/models.py:250-264).
_LAYER_SMALL = dict(B=1, T=32, hidden=128, head_dim=32, q_out=128, kv_out=32, intermediate=352)
_LAYER_SMALL_2 = dict(B=2, T=17, hidden=64, head_dim=16, q_out=64, kv_out=16, intermediate=176)


def _llama3_8b_layer(tokens: int) -> dict:
    return dict(B=1, T=tokens, hidden=4096, head_dim=128, q_out=4096, kv_out=1024,
                intermediate=14336)


def _layer_tokens_feature(workload) -> float:
    return float(workload.dims["B"] * workload.dims["T"])


LLAMA3_DECODER_LAYER = declare_op(
    name="llama3_decoder_layer",
    forward="oracle.forward_refs:llama3_decoder_layer_forward_ref",
    runtime_forward="oracle.forward_refs:llama3_decoder_layer_runtime_ref",
    reference_dtype="float32",
    dims=("B", "T", "hidden", "head_dim", "q_out", "kv_out", "intermediate"),
    args=(
        Active("x", "[B, T, hidden]"),
        Active("input_norm_weight", "[hidden]", note="RMSNorm gain before attention"),
        Active("q_weight", "[q_out, hidden]"),
        Active("k_weight", "[kv_out, hidden]", note="fewer heads than q under GQA"),
        Active("v_weight", "[kv_out, hidden]"),
        Active("o_weight", "[hidden, q_out]"),
        Active("post_norm_weight", "[hidden]", note="RMSNorm gain before the MLP"),
        Active("gate_weight", "[intermediate, hidden]"),
        Active("up_weight", "[intermediate, hidden]"),
        Active("down_weight", "[hidden, intermediate]"),
        Inactive("cos", "[T, head_dim]", note="rotary table, duplicated halves"),
        Inactive("sin", "[T, head_dim]", note="rotary table, duplicated halves"),
        Inactive("eps", default=1e-5),
    ),
    output=Active("out", "[B, T, hidden]"),
    forward_semantics=(
        "One Llama-3 decoder layer over x [batch, tokens, hidden]: RMSNorm -> Q/K/V "
        "projections -> half-rotated RoPE on Q and K -> causal grouped-query attention -> "
        "output projection -> residual add -> RMSNorm -> SwiGLU MLP (silu(gate) * up, then "
        "down) -> residual add. Weights in nn.Linear [out, in] orientation; head counts "
        "q_out // head_dim and kv_out // head_dim. RMSNorm statistics, the SiLU and the "
        "attention softmax in fp32; causal; no KV cache, no dropout."
    ),
    backward_semantics=(
        "Gradients of all ten Active inputs in declaration order: dx, dinput_norm_weight, "
        "dq_weight, dk_weight, dv_weight, do_weight, dpost_norm_weight, dgate_weight, "
        "dup_weight, ddown_weight; dx accumulates the two residual paths and the norm "
        "inputs; key/value gradients summed over each query group; reductions in fp32."
    ),
    correctness=(
        Workload(dims=_LAYER_SMALL, dtype="float32", atol=1e-4, rtol=1e-4),
        Workload(dims=_LAYER_SMALL_2, dtype="float32", atol=1e-4, rtol=1e-4),
        Workload(dims=_LAYER_SMALL, dtype="bfloat16"),
        Workload(dims=_LAYER_SMALL_2, dtype="bfloat16"),
    ),
    benchmark=tuple(
        Workload(dims=_llama3_8b_layer(t), dtype="bfloat16", label=f"llama3_8b_T{t}")
        for t in (1024, 2048, 4096)
    ),
    tolerances={"float32": (1e-4, 1e-4), "bfloat16": (5e-2, 2e-2)},
    tolerance_multipliers={
        "dk_weight": (1.5, 1.0),
        "dv_weight": (1.5, 1.0),
        "ddown_weight": (1.5, 1.0),
    },
    make_inputs="evograd_amd.inputs:make_llama3_decoder_layer_inputs",
    memory_inputs=("x", "input_norm_weight", "q_weight", "k_weight", "v_weight", "o_weight",
                   "post_norm_weight", "gate_weight", "up_weight", "down_weight"),
    regime_feature=_layer_tokens_feature,
    regime_split=LLAMA_REGIME_SPLIT,
)

OPS: dict[str, OpDecl] = {
    op.name: op
    for op in (SOFTMAX, RMSNORM, LAYERNORM, SWIGLU, ROPE, CAUSAL_ATTENTION, FUSED_ADD_RMS_NORM,
               CAUSAL_ATTENTION_GQA, LLAMA3_ATTENTION, CROSS_ENTROPY, FUSED_LINEAR_CROSS_ENTROPY,
               LLAMA3_DECODER_LAYER)
}


def get_op(name: str) -> OpDecl:
    """Look up a declaration by name (src/evograd/ops/__init__.py:90-99)."""
    try:
        return OPS[name]
    except KeyError:
        raise KeyError(f"unknown op {name!r}; known: {sorted(OPS)}") from None
