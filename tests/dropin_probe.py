"""Helper module run inside a child process by tests/test_dropin.py (not a test file itself).

The child is started the way the reference's int8_runtime._spawn starts its self-test child
(int8_runtime.py:292, 501-524): argv[1] is the parent's ``sys.path`` as JSON, prepended before any
import, argv[2] the module to import with importlib, argv[3] the shapes as JSON, argv[4] the device and
argv[5] the backend; the module's ``selftest(shapes, device, backend)`` result is printed as the last line
of stdout, as JSON.  ``selftest`` here reports what the bare names ``int8_kernels`` and ``fused_kernels``
resolved to in the child and, on a GPU device, runs mica_amd's self-test through the module so resolved.
"""
import sys


def selftest(shapes, device, backend="aot"):
    import int8_kernels as aot      # the bare names the reference's modules import
    import fused_kernels as ffk

    import mica_amd.fused_kernels
    import mica_amd.int8_kernels

    stats = aot.kernel_dir() / "s.pt"
    out = {
        "int8_kernels": aot.__name__,
        "fused_kernels": ffk.__name__,
        "same_int8_kernels": aot is mica_amd.int8_kernels,
        "same_fused_kernels": ffk is mica_amd.fused_kernels,
        "same_stats": aot.STATS is mica_amd.int8_kernels.STATS,
        "int8_kernels_file": sys.modules["int8_kernels"].__file__,
        "stats_path": str(stats),
        "stats_found": stats.is_file(),
        "lib_dir": str(aot.lib_dir()),
    }
    if out["stats_found"]:
        from mica_amd import int8_runtime

        out["stats_entries"] = len(int8_runtime.load_stats(stats))
    if device.startswith("cuda"):
        from mica_amd import int8_runtime

        launches = aot.STATS["launch"]
        out["selftest"] = int8_runtime.selftest([tuple(s) for s in shapes], device, backend)
        out["launches_seen_by_int8_kernels"] = aot.STATS["launch"] - launches
    return out
