"""The C-ABI library loads and exports every entry point include/gg.h declares
(no compute: this runs without a GPU)."""
import ctypes
import os
import re

from gemma_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "gg.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b(gg_[a-z0-9_]+)\s*\(", src)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ["gg_create", "gg_upload_tensor", "gg_finalize", "gg_prefill", "gg_select", "gg_step",
              "gg_penalty_reset", "gg_penalty_add", "gg_reset_kv", "gg_read", "gg_last_error", "gg_destroy"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(capi.LIB_PATH)
    for n in declared_functions():
        assert hasattr(lib, n), n
    # the Python mirror binds exactly the declared set
    assert sorted(capi.exported_symbols()) == declared_functions()


def test_struct_layouts_match_header():
    assert ctypes.sizeof(capi.GGConfig) == 15 * 4
    assert ctypes.sizeof(capi.GGSample) == 3 * 8


def test_create_rejects_bad_config_without_touching_a_device():
    cfg = capi.GGConfig(1152, 26, 4, 1, 128, 6912, 262144, 2048, 1e-6, 1e6, 1e6, 6, 0, 0, 0)  # head_dim 128
    lib = capi.lib()
    assert not lib.gg_create(ctypes.byref(cfg))
    assert b"head_dim" in lib.gg_last_error(None)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 exits with status 2 and says
    why, before anything touches a device."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
