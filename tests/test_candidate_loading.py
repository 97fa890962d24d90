"""Every pair module is a drop-in candidate file: it loads the way evograd's commands
load a program -- a fresh interpreter, any working directory, the package not on
sys.path, ``spec_from_file_location("evograd_candidate_<stem>", path)``
(src/evograd/opdecl/verify_cli.py:22-28; the bench CLIs and the emitted
dispatcher load the same way) -- and the declaration's pair is then found in it.
No GPU call is made: loading a pair module opens nothing native."""

import json
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

from evograd_amd import PAIR_MODULES

ROOT = Path(__file__).resolve().parents[1]

# pair-module file -> declarations it serves
PAIR_FILES = {}
for _op, _mod in PAIR_MODULES.items():
    PAIR_FILES.setdefault(ROOT / (_mod.replace(".", "/") + ".py"), []).append(_op)


def _run_isolated(script: str, tmp_path) -> dict:
    """Run ``script`` in a fresh interpreter from ``tmp_path`` with the repository
    absent from sys.path; the script prints one JSON line."""
    env = {"PATH": "/usr/bin:/bin", "HOME": str(tmp_path), "PYTHONNOUSERSITE": "1"}
    proc = subprocess.run([sys.executable, "-c", script], cwd=tmp_path, env=env,
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-3000:]
    return json.loads(proc.stdout.strip().splitlines()[-1])


LOAD_AND_LOOKUP = textwrap.dedent('''
    import importlib.util, json, sys
    from pathlib import Path
    assert not any(Path(p or ".").resolve() == Path({root!r}) for p in sys.path)
    path = Path({path!r})
    spec = importlib.util.spec_from_file_location(f"evograd_candidate_{{path.stem}}", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    from evograd_amd.bind import lookup_pair
    from evograd_amd.decls import get_op
    found = {{}}
    for op_name in {ops!r}:
        fwd, bwd = lookup_pair(get_op(op_name), module)
        found[op_name] = [fwd.__name__, bwd.__name__, fwd.__module__]
    print(json.dumps(found))
''')


@pytest.mark.parametrize("path", sorted(PAIR_FILES), ids=lambda p: p.stem)
def test_pair_file_loads_as_a_top_level_candidate(path, tmp_path):
    ops = PAIR_FILES[path]
    found = _run_isolated(LOAD_AND_LOOKUP.format(root=str(ROOT), path=str(path), ops=ops),
                          tmp_path)
    for op_name in ops:
        fwd, bwd, module = found[op_name]
        assert fwd == f"{op_name}_forward_with_saved"
        assert bwd == f"{op_name}_backward_from_saved"
        assert module == f"evograd_candidate_{path.stem}"


def _extra_files():
    from evograd_amd import DISPATCH_MODULES, SMALL_PROGRAMS

    for table in (SMALL_PROGRAMS, DISPATCH_MODULES):
        for op_name, mod in sorted(table.items()):
            yield pytest.param(op_name, ROOT / (mod.replace(".", "/") + ".py"),
                               id=mod.rsplit(".", 1)[1])


@pytest.mark.parametrize("op_name,path", list(_extra_files()))
def test_small_programs_and_dispatchers_load_as_candidates(op_name, path, tmp_path):
    """The small-shape programs and the dispatchers over them load from their paths
    like any candidate, with the repository off sys.path, and expose the pair."""
    found = _run_isolated(LOAD_AND_LOOKUP.format(root=str(ROOT), path=str(path), ops=[op_name]),
                          tmp_path)
    fwd, bwd, _ = found[op_name]
    assert fwd.endswith("forward_with_saved") and bwd.endswith("backward_from_saved")


def test_every_declaration_has_a_pair_file():
    from evograd_amd.decls import OPS

    assert sorted(OPS) == sorted(PAIR_MODULES)
    for path in PAIR_FILES:
        assert path.is_file(), path


EMIT_AND_LOAD = textwrap.dedent('''
    import importlib.util, json, sys
    sys.path.insert(0, {root!r})
    from evograd_amd.decls import get_op
    from evograd_amd.dispatch import emit_dispatcher
    out = emit_dispatcher(get_op("rmsnorm"), {small!r}, {large!r}, 16.0, {out!r})
    sys.path.remove({root!r})
    for name in [m for m in sys.modules if m.startswith("evograd_amd")]:
        del sys.modules[name]
    spec = importlib.util.spec_from_file_location("evograd_candidate_dispatch", out)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    pair = module._DISPATCH
    print(json.dumps([type(p).__name__ for p in pair.programs] +
                     [m.__name__ for m in pair.programs] +
                     [hasattr(module, "rmsnorm_forward_with_saved"),
                      hasattr(module, "rmsnorm_backward_from_saved")]))
''')


def test_emitted_dispatcher_over_hip_pair_files_loads(tmp_path):
    rms = str(ROOT / "evograd_amd" / "pairs" / "rmsnorm.py")
    got = _run_isolated(EMIT_AND_LOAD.format(root=str(ROOT), small=rms, large=rms,
                                             out=str(tmp_path / "dispatch_rmsnorm.py")),
                        tmp_path)
    assert got == ["module", "module", "evograd_dispatch_small_rmsnorm",
                   "evograd_dispatch_large_rmsnorm", True, True]
