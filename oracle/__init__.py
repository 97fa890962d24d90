"""CPU-checkable oracle for the autograd-pair hot path — TEST INFRASTRUCTURE ONLY.

This package restates the reference's ground truth: each operator's trusted
PyTorch forward (the ``forward_ref.py`` files of src/evograd/ops/) differentiated
by ``torch.autograd.grad`` (src/evograd/opdecl/oracle.py:44-111) and the
correctness gate (src/evograd/opdecl/verify.py:85-160). The seeded input recipes
(src/evograd/opdecl/inputs.py) are harness code shared with the benchmark and
live in ``evograd_amd.inputs``.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import it, and only as the checker or the timed CPU baseline. The product
(``evograd_amd``) never imports it: its pair modules call the HIP library and
fail loudly when it is missing.

The reference's arithmetic lives in PyTorch (a third-party dependency, unpinned in
the reference's pyproject.toml:13-17; installed here as torch 2.10.0+rocm7.0), so
the oracle is a torch restatement rather than a C one. How each function is pinned
(closed forms, invariants, fp64 finite differences, brute force on tiny inputs)
is recorded in tests/test_oracle_pins.py; no function of this package is left
unpinned.
"""
