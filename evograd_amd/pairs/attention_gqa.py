"""Grouped-query causal attention pair (k, v with fewer heads than q).

The kernels and calls are those of ``evograd_amd.pairs.attention``, which takes
k and v of [B, Hkv, S, D] for any Hkv dividing H; this module gives them the
names the ``causal_attention_gqa`` declaration looks up
(src/evograd/opdecl/bind.py:28-47 resolves ``<op>_forward_with_saved``).
"""

from __future__ import annotations

from .attention import causal_attention_backward_from_saved, causal_attention_forward_with_saved

causal_attention_gqa_forward_with_saved = causal_attention_forward_with_saved
causal_attention_gqa_backward_from_saved = causal_attention_backward_from_saved
