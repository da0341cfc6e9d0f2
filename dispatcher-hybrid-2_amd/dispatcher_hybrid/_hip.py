"""ctypes binding of libdh_mixer.so, the gfx950 kernels behind the fused paths.

The library exposes a plain C ABI (``include/dh_mixer.h`` at the repository root): device
pointers, sizes and a ``hipStream_t``. This module loads it after ``torch`` (so the library binds
to the HIP runtime torch already mapped), declares every entry point's signature, and turns a
non-zero status into a Python exception carrying the library's message.

There is no fallback: if the library is missing or fails to load, importing this module raises
``ImportError`` (the same failure the reference's fused modules give when Triton is absent,
reference dispatcher_hybrid/fused_gates.py:33-35, dispatcher_hybrid/decoding.py:452-453).
"""

import ctypes
import os

import torch

ABI_VERSION = 19
_LIB_NAME = "libdh_mixer.so"

DH_F32, DH_BF16 = 0, 1
_STATUS = {
    1: ("INVALID_ARG", ValueError),
    2: ("UNSUPPORTED_SHAPE", ValueError),
    3: ("UNSUPPORTED_DTYPE", TypeError),
    4: ("LAUNCH_FAILED", RuntimeError),
    5: ("UNIMPLEMENTED", NotImplementedError),
}


def library_path():
    """Path of the kernel library: $DH_MIXER_LIB, else the in-tree build under ``_lib/``."""
    env = os.environ.get("DH_MIXER_LIB")
    if env:
        return env
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", _LIB_NAME)


def _load():
    path = library_path()
    if not os.path.isfile(path):
        raise ImportError(
            f"{_LIB_NAME} not found at {path}; build it first "
            "(python -c 'import __graft_entry__ as g; g.build()' from the repository root, "
            "or python -m dispatcher_hybrid._build)")
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:  # pragma: no cover - depends on the host
        raise ImportError(f"cannot load {path}: {e}") from e
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    sigs = {
        "dh_abi_version": ([], i32),
        "dh_last_error": ([], ctypes.c_char_p),
        "dh_gate_preacts_fwd": ([i32, vp, vp, i64, i64, vp, vp, vp, i64, i64, vp, vp, vp,
                                 vp, i64, i64, i64, vp, vp, vp, i64, i64, i64, i64,
                                 i32, i32, i32, i32, i32, i32, vp], i32),
        "dh_gate_preacts_bwd": ([i32, vp, vp, i64, i64, vp, vp, vp, i64, i64, vp, vp, vp,
                                 vp, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp,
                                 i32, i32, i32, i32, i32, vp], i32),
        "dh_level_scan_fwd": ([i32, vp, vp, vp, i64, i64, i64, i64, vp, i64, i64, i64,
                               vp, i64, i64, vp, i32, i32, i32, i32, i32, i32, vp, i32, vp], i32),
        "dh_decode_mixer_step": ([i32] + [vp] * 13 + [i32] * 7 + [vp], i32),
        "dh_step_gates": ([i32] + [vp] * 12 + [i32] * 5 + [vp], i32),
        "dh_decode_gemv": ([i32, vp, i64, vp, vp, ctypes.c_float, i32, vp, vp, vp, vp, vp,
                            vp, i64, vp, i32, vp, vp, vp, i32, i32, vp], i32),
        "dh_decode_gemv_candidates": ([i32, i32, i32], i64),
        "dh_argmax_reduce": ([vp, i32, i32, vp, vp, vp, i64, i64, vp], i32),
        "dh_step_scan": ([i32] + [vp] * 7 + [i32] * 6 + [vp], i32),
        "dh_decode_attention": ([i32, vp, vp, vp, i64, vp, vp, vp, vp, vp, vp, i64,
                                 i32, i32, i32, i32, i32, vp], i32),
        "dh_argmax": ([i32, vp, i64, i32, i32, vp, vp, i64, vp], i32),
        "dh_argmax_noalloc": ([i32, vp, i64, i32, i32, vp, vp], i32),
        "dh_decode_attention_workspace_bytes": ([i32, i32, i32], i64),
        "dh_decode_attention_split": ([i32, vp, vp, vp, i64, vp, vp, vp, vp, vp, vp, i64, i32, i32, i32, i32, i32,
                                       vp, i64, vp], i32),
        "dh_window_attention_fwd": ([i32, vp, vp, vp, i64, i64, vp, vp, vp, i64, i64, vp, vp, i64, i64,
                                     i32, i32, i32, i32, i32, i32, vp], i32),
        "dh_decode_scan_out": ([i32] + [vp] * 8 + [i64, vp] + [i32] * 6 + [vp], i32),
        "dh_proj_gemm": ([i32, vp, i64, i32, i32, i32, vp, vp, vp, vp, vp], i32),
        "dh_proj_gemm_swiglu": ([i32, vp, i64, i32, i32, vp, vp, i32, vp, i64, vp], i32),
        "dh_tree_mask": ([i32, vp, i64, i32, i32, i32, i64, vp, vp], i32),
        "dh_sample_topk": ([i32, vp, i64, i32, i32, ctypes.c_float, i32, ctypes.c_uint64, vp, vp, vp], i32),
        "dh_sample_topk_hist": ([i32, vp, i64, i32, i32, ctypes.c_float, i32, ctypes.c_uint64, vp, vp, vp, i64, i64,
                                 vp], i32),
        "dh_argmax_workspace_bytes": ([i32, i32], i64),
        "dh_decode_gates": ([i32] + [vp] * 12 + [i32] * 7 + [vp], i32),
        "dh_decode_scan": ([i32] + [vp] * 5 + [i32] * 6 + [vp], i32),
        "dh_decode_persistent_scratch_bytes": ([i32] * 6, i64),
        "dh_decode_persistent_step": ([vp, vp, i32, vp, vp, ctypes.c_float] + [i32] * 8
                                      + [vp, vp, vp, i64, vp, vp, i64, vp], i32),
        "dh_decode_persistent_status": ([vp, vp, vp], i32),
        "dh_decode_persistent_trace": ([vp, vp, i32, vp, vp, ctypes.c_float] + [i32] * 8
                                       + [vp, vp, vp, i64, vp, vp, i64, vp, i64, vp], i32),
        "dh_decode_persistent_phases": ([vp, i32], i32),
        "dh_silu_mul": ([i32, vp, vp, vp, i64, vp], i32),
        "dh_add_rmsnorm": ([i32, vp, vp, vp, ctypes.c_float, vp, vp, i64, i32, vp], i32),
    }
    for name, (argtypes, restype) in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    ver = lib.dh_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f"{path} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
    return lib


lib = _load()


def check(status, what):
    """Raise the exception mapped to a non-zero dh_status."""
    if status == 0:
        return
    name, exc = _STATUS.get(status, ("UNKNOWN", RuntimeError))
    msg = lib.dh_last_error().decode(errors="replace")
    raise exc(f"{what} failed ({name}): {msg}")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device=None):
    """hipStream_t of torch's current stream on `device` (the capture stream under graph capture)."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype):
    if dtype == torch.float32:
        return DH_F32
    if dtype == torch.bfloat16:
        return DH_BF16
    raise TypeError(f"dispatcher kernels support float32 and bfloat16, got {dtype}")


def require_gpu(t, what):
    if not t.is_cuda:
        raise RuntimeError(f"{what}: tensors must be on the GPU (got device {t.device}); "
                           "the fused paths have no CPU implementation")
