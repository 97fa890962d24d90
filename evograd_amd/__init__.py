"""evograd_amd: gfx950 (MI355X) HIP kernels behind evograd's autograd-pair hot path.

Layout:

* ``csrc/``     HIP sources of libevograd_hip.so (C ABI in include/evograd_hip.h)
* ``_lib``      ctypes binding of that library (no CPU fallback)
* ``opdecl``    the torch-free declaration contract (Active, Inactive, Workload, OpDecl)
* ``decls``     declarations of softmax, rmsnorm, layernorm, swiglu, rope, causal_attention,
                fused_add_rms_norm, causal_attention_gqa, llama3_attention (RoPE on q, k
                then grouped causal attention), cross_entropy, fused_linear_cross_entropy,
                llama3_decoder_layer (one whole Llama-3 decoder layer)
* ``pairs``     one module per operator with the reference's
                ``<op>_forward_with_saved`` / ``<op>_backward_from_saved`` functions
* ``bind``      ``bind(op, module)`` -> a ``torch.autograd.Function``-backed callable
* ``harness``   saved-state accounting and device timing used by the benchmark
"""

__version__ = "0.1.0"

PAIR_MODULES = {
    "softmax": "evograd_amd.pairs.softmax",
    "rmsnorm": "evograd_amd.pairs.rmsnorm",
    "layernorm": "evograd_amd.pairs.layernorm",
    "swiglu": "evograd_amd.pairs.swiglu",
    "rope": "evograd_amd.pairs.rope",
    "causal_attention": "evograd_amd.pairs.attention",
    "fused_add_rms_norm": "evograd_amd.pairs.fused_add_rms_norm",
    "causal_attention_gqa": "evograd_amd.pairs.attention_gqa",
    "llama3_attention": "evograd_amd.pairs.llama3_attention",
    "cross_entropy": "evograd_amd.pairs.cross_entropy",
    "fused_linear_cross_entropy": "evograd_amd.pairs.fused_linear_cross_entropy",
    "llama3_decoder_layer": "evograd_amd.pairs.llama3_decoder_layer",
}

# Small-shape programs and the shape dispatchers that route to them below the
# declaration's regime split (the registered PAIR_MODULES program above it).
SMALL_PROGRAMS = {
    "rmsnorm": "evograd_amd.pairs.rmsnorm_small",
    "layernorm": "evograd_amd.pairs.layernorm_small",
}
DISPATCH_MODULES = {
    "rmsnorm": "evograd_amd.pairs.rmsnorm_dispatch",
    "layernorm": "evograd_amd.pairs.layernorm_dispatch",
}


def dispatch_module(op_name: str):
    """The shape-dispatched pair of ``op_name`` (KeyError when it has none)."""
    import importlib

    return importlib.import_module(DISPATCH_MODULES[op_name])


def pair_module(op_name: str):
    """Import the HIP-backed pair module for ``op_name``."""
    import importlib

    try:
        return importlib.import_module(PAIR_MODULES[op_name])
    except KeyError:
        raise KeyError(f"no pair module for {op_name!r}; known: {sorted(PAIR_MODULES)}") from None
