"""HIP-backed autograd pairs, one module per operator.

Each module exposes ``<op>_forward_with_saved`` and ``<op>_backward_from_saved``
with the argument lists of the reference declarations, so it is looked up by
``lookup_pair`` exactly like a reference candidate module. Every function
launches kernels from libevograd_hip.so on torch's current stream and returns
without synchronising.
"""
