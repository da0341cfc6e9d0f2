"""C-ABI boundary: the library loads, exports every entry point include/dh_mixer.h declares, and
rejects bad arguments with its status codes before touching the device (no GPU needed)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dh_mixer.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(dh_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("dh_abi_version", "dh_last_error", "dh_gate_preacts_fwd", "dh_gate_preacts_bwd",
                 "dh_level_scan_fwd", "dh_decode_mixer_step", "dh_decode_gemv", "dh_decode_attention", "dh_argmax",
                 "dh_decode_gates", "dh_decode_scan", "dh_argmax_workspace_bytes", "dh_sample_topk", "dh_sample_topk_hist", "dh_proj_gemm", "dh_proj_gemm_swiglu", "dh_tree_mask", "dh_decode_scan_out", "dh_decode_attention_split",
                 "dh_decode_attention_workspace_bytes", "dh_window_attention_fwd",
                 "dh_step_gates", "dh_step_scan"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from dispatcher_hybrid import _hip
    lib = ctypes.CDLL(_hip.library_path())
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in dh_mixer.h but not exported"
    assert _hip.lib.dh_abi_version() == _hip.ABI_VERSION


def test_status_codes_without_device_work():
    from dispatcher_hybrid import _hip
    lib = _hip.lib
    S = None
    # unsupported dtype
    st = lib.dh_decode_mixer_step(7, *([S] * 13), 1, 8, 14, 64, 2, 64, 3, S)
    assert st == 3 and b"dtype" in lib.dh_last_error()
    # unsupported head width
    st = lib.dh_decode_mixer_step(1, *([S] * 13), 1, 8, 14, 64, 2, 48, 3, S)
    assert st == 2 and b"hd=48" in lib.dh_last_error()
    # S inconsistent with L
    st = lib.dh_decode_mixer_step(1, *([S] * 13), 1, 8, 13, 64, 2, 64, 3, S)
    assert st == 1
    # null pointers
    st = lib.dh_decode_mixer_step(1, *([S] * 13), 1, 8, 14, 64, 2, 64, 3, S)
    assert st == 1 and b"null" in lib.dh_last_error()
    st = lib.dh_gate_preacts_fwd(0, *([S] * 2), 0, 0, *([S] * 3), 0, 0, *([S] * 4), 0, 0, 0,
                                 *([S] * 3), 0, 0, 0, 0, 0, 1, 8, 60, 2, 3, S)
    assert st == 2 and b"GH=60" in lib.dh_last_error()
    st = lib.dh_level_scan_fwd(1, *([S] * 3), 0, 0, 0, 0, S, 0, 0, 0, S, 0, 0, S, 1, 40000, 2, 64, 3, 0, S, 0, S)
    assert st == 2 and b"32768" in lib.dh_last_error()
    st = lib.dh_level_scan_fwd(1, *([S] * 3), 0, 0, 0, 0, S, 0, 0, 0, S, 0, 0, S, 1, 64, 2, 64, 3, 1, S, 0, S)
    assert st == 1 and b"null" in lib.dh_last_error()


def test_python_wrapper_maps_status_to_exceptions():
    from dispatcher_hybrid import _hip
    with pytest.raises(TypeError, match="UNSUPPORTED_DTYPE"):
        _hip.check(3, "x")
    with pytest.raises(ValueError, match="INVALID_ARG"):
        _hip.check(1, "x")
    with pytest.raises(RuntimeError, match="LAUNCH_FAILED"):
        _hip.check(4, "x")
    _hip.check(0, "x")


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    """No fallback: pointing the loader at a missing library raises ImportError."""
    import importlib.util
    import sys
    monkeypatch.setenv("DH_MIXER_LIB", str(tmp_path / "nope.so"))
    spec = importlib.util.spec_from_file_location(
        "dh_hip_probe", os.path.join(ROOT, "dispatcher-hybrid-2_amd", "dispatcher_hybrid", "_hip.py"))
    mod = importlib.util.module_from_spec(spec)
    with pytest.raises(ImportError, match="not found"):
        spec.loader.exec_module(mod)
    sys.modules.pop("dh_hip_probe", None)
