"""The pair files, loaded as evograd loads a candidate (a top-level module executed
from its path, src/evograd/opdecl/verify_cli.py:22-28), pass the gate on the GPU:
one correctness workload per declaration, plus a dispatcher module emitted over
two HIP pair files and loaded the same way."""

import sys
from pathlib import Path

import pytest
import torch

from evograd_amd import PAIR_MODULES, decls
from evograd_amd.dispatch import emit_dispatcher, load_module
from oracle.verify import verify

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _file_of(op_name: str) -> Path:
    return ROOT / (PAIR_MODULES[op_name].replace(".", "/") + ".py")


@pytest.mark.parametrize("op_name", sorted(PAIR_MODULES))
def test_path_loaded_candidate_passes_the_gate(op_name):
    op = decls.get_op(op_name)
    w = op.correctness[0]
    print(f"\n[gpu-candidate] {op_name} {w.dims} {w.dtype}", flush=True)
    module = load_module(_file_of(op_name))
    assert module.__name__.startswith("evograd_candidate_")
    rep = verify(op, module, device="cuda", workloads=(w,))
    torch.cuda.synchronize()
    assert rep.ok, "\n".join(rep.failures())


def test_emitted_dispatcher_over_hip_files_passes_the_gate(tmp_path):
    """A dispatcher module written to disk over two different program files (the
    small-shape program and the ring program), loaded by path as a candidate."""
    from evograd_amd import SMALL_PROGRAMS

    op = decls.RMSNORM
    rms = _file_of("rmsnorm")
    small_file = ROOT / (SMALL_PROGRAMS["rmsnorm"].replace(".", "/") + ".py")
    out = emit_dispatcher(op, small_file, rms, 64.0, tmp_path / "dispatch_rmsnorm.py")
    module = load_module(out)
    small = [w for w in op.correctness if w.dims["rows"] < 64][:1]
    large = [w for w in op.correctness if w.dims["rows"] >= 64][:1]
    assert small and large
    print(f"\n[gpu-candidate] dispatcher {small[0].dims} {large[0].dims}", flush=True)
    sys.stdout.flush()
    rep = verify(op, module, device="cuda", workloads=(*small, *large))
    assert rep.ok, "\n".join(rep.failures())
    x = torch.randn(80, 256, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(256, device="cuda", dtype=torch.bfloat16)
    _, saved = module.rmsnorm_forward_with_saved(x, w, 1e-6)
    assert saved[0] == 1 and isinstance(saved[0], int)
    _, saved = module.rmsnorm_forward_with_saved(x[:8], w, 1e-6)
    assert saved[0] == 0
