"""The drop-in directory ``mica_amd/dropin`` across the reference's start-up sequence.

The reference's server imports ``int8_kernels`` / ``fused_kernels`` by bare name, and runs its
acceptance self-test in a child process that rebuilds the parent's ``sys.path`` and imports the module
again from scratch (int8_runtime.py:292, 501-524).  The convert route then looks for the SmoothQuant
statistics at ``int8_kernels.kernel_dir() / 's.pt'`` (int8_runtime.py:227, 265; MICA_W8A8_AOT_DIR,
int8_kernels.py:83-84).  These tests start a child the same way (JSON ``sys.path`` in argv, then
``importlib.import_module``), with the drop-in directory first on the path, and check what the names
resolve to there.  None of them imports or runs the reference's code.
"""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
DROPIN = ROOT / "mica_amd" / "dropin"
TESTS = ROOT / "tests"

# the child's program: prepend the parent's search path, import the named module, call its
# selftest(shapes, device, backend) and print the result as the last line
CHILD = (
    "import json, sys\n"
    "sys.path[:0] = json.loads(sys.argv[1])\n"
    "import importlib\n"
    "mod = importlib.import_module(sys.argv[2])\n"
    "res = mod.selftest([tuple(s) for s in json.loads(sys.argv[3])], sys.argv[4], sys.argv[5])\n"
    "sys.stdout.write('\\n' + json.dumps(res) + '\\n')\n"
)


def spawn(module, shapes, device, env_extra=None, timeout=300):
    """Start the child as the reference's _spawn does and return its JSON result."""
    search = [str(DROPIN), str(TESTS)] + [p for p in sys.path if p not in (str(ROOT), "")]
    env = dict(os.environ)
    env.pop("MICA_W8A8_AOT_DIR", None)
    env.update(env_extra or {})
    proc = subprocess.run([sys.executable, "-B", "-c", CHILD, json.dumps(search), module, json.dumps(shapes),
                           device, "aot"], capture_output=True, text=True, timeout=timeout, env=env,
                          cwd=str(TESTS))
    assert proc.returncode == 0, proc.stderr[-3000:]
    return json.loads(proc.stdout.strip().splitlines()[-1])


def write_stats(folder):
    """A small statistics file in the reference's packed layout: h (name keys), o (offsets), v (values)."""
    from mica_amd.int8_runtime import name_key

    keys = torch.tensor([name_key("layers.0.mlp.gate_proj"), name_key("layers.0.mlp.up_proj")], dtype=torch.int64)
    torch.save({"h": keys, "o": torch.tensor([0, 4, 8]), "v": torch.arange(8, dtype=torch.float32)},
               str(folder / "s.pt"))


def test_child_resolves_bare_names_to_mica_amd(tmp_path):
    write_stats(tmp_path)
    r = spawn("dropin_probe", [], "cpu", {"MICA_W8A8_AOT_DIR": str(tmp_path)})
    assert r["int8_kernels"] == "mica_amd.int8_kernels"
    assert r["fused_kernels"] == "mica_amd.fused_kernels"
    assert r["same_int8_kernels"] and r["same_fused_kernels"] and r["same_stats"]
    assert Path(r["int8_kernels_file"]).resolve() == (ROOT / "mica_amd" / "int8_kernels.py").resolve()
    assert Path(r["stats_path"]) == tmp_path / "s.pt" and r["stats_found"]
    assert r["stats_entries"] == 2
    assert Path(r["lib_dir"]).resolve() == (ROOT / "mica_amd").resolve()


def test_child_without_stats_dir_uses_library_dir():
    r = spawn("dropin_probe", [], "cpu")
    assert Path(r["stats_path"]).parent.resolve() == (ROOT / "mica_amd").resolve()
    assert not r["stats_found"]


def test_kernel_dir_follows_env(monkeypatch, tmp_path):
    from mica_amd import int8_kernels

    monkeypatch.setenv("MICA_W8A8_AOT_DIR", str(tmp_path))
    assert int8_kernels.kernel_dir() == tmp_path
    monkeypatch.delenv("MICA_W8A8_AOT_DIR")
    assert int8_kernels.kernel_dir() == int8_kernels.lib_dir()


def test_shim_in_this_process_is_the_package_module(monkeypatch):
    import importlib

    from mica_amd import fused_kernels, int8_kernels

    monkeypatch.syspath_prepend(str(DROPIN))
    for name in ("int8_kernels", "fused_kernels"):
        monkeypatch.delitem(sys.modules, name, raising=False)
    assert importlib.import_module("int8_kernels") is int8_kernels
    assert importlib.import_module("fused_kernels") is fused_kernels


@pytest.mark.gpu
def test_selftest_in_spawned_child(gpu):
    """The acceptance self-test, run in a child started as the reference starts it, through the bare
    module names: every QLinear call takes 2 launches and meets the 1.05 x INT8-noise bound."""
    print("[case] self-test in a spawned child", file=sys.stderr, flush=True)
    shapes = [(32, 2560, False), (1024, 2560, True), (2560, 4096, False)]
    r = spawn("dropin_probe", shapes, f"cuda:{gpu.index}")
    assert r["same_int8_kernels"] and r["same_fused_kernels"], r
    st = r["selftest"]
    assert st["ok"], st
    assert st["cases"] == len(shapes) * 2 * 5          # smoothed and not, 5 row counts each
    assert st["kernel_launches"] == 2 * st["cases"]
    assert r["launches_seen_by_int8_kernels"] == st["kernel_launches"]
