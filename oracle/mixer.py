"""TEST INFRASTRUCTURE ONLY — float64 checker for the mixer kernels.

numpy front end of the C restatement in dh_oracle.c (built by oracle/build.py), plus the integer
mask and ring-slot arithmetic in numpy. Only tests/, __graft_entry__.smoke() and bench.py's CPU
baseline import this; the product never does.

Reference semantics followed (file:line in /root/reference):
  ring_offset / ring_slot   dispatcher_hybrid/decoding.py:59-66, fused_step.py:81-86
  level_mask                dispatcher_hybrid/modeling_dispatcher.py:282-297
  tree_mask                 dispatcher_hybrid/modeling_dispatcher.py:311-323
  gate_preacts              dispatcher_hybrid/modeling_dispatcher.py:100-109, fused_gates.py:38-93
  level_scan                dispatcher_hybrid/modeling_dispatcher.py:86-88, 111-121
  decode_step               dispatcher_hybrid/fused_step.py:26-88, decoding.py:187-222
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libdh_oracle.so")
_lib = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.isfile(_LIB_PATH):
            from . import build
            build.build()
        lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.POINTER(ctypes.c_double)
        i32, i64 = ctypes.c_int, ctypes.c_int64
        lib.dh_oracle_ring_offset.argtypes = [i32]
        lib.dh_oracle_ring_offset.restype = i64
        lib.dh_oracle_ring_slot.argtypes = [i32, i64]
        lib.dh_oracle_ring_slot.restype = i64
        lib.dh_oracle_gate_preacts.argtypes = [P] * 9 + [i32] + [P] * 3 + [i32] * 6
        lib.dh_oracle_gate_preacts.restype = None
        lib.dh_oracle_level_scan.argtypes = [P] * 4 + [i32] + [P] * 3 + [i32] * 5
        lib.dh_oracle_level_scan.restype = None
        lib.dh_oracle_decode_step.argtypes = [P] * 8 + [i64] + [P] * 4 + [i32] * 7
        lib.dh_oracle_decode_step.restype = None
        _lib = lib
    return _lib


def _f64(x):
    return np.ascontiguousarray(np.asarray(x, dtype=np.float64))


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def ring_offset(j):
    return int(_load().dh_oracle_ring_offset(j))


def ring_slot(j, p):
    return int(_load().dh_oracle_ring_slot(j, p))


def ring_slots_numpy(j, p):
    """Vectorised ring slot for an integer array of positions."""
    p = np.asarray(p, dtype=np.int64)
    return ((1 << (j + 1)) - 2) + (p & ((1 << (j + 1)) - 1))


def level_mask(T, L):
    """(T, L) float64: 1 where t >= 2^l (and 2^l < T)."""
    t = np.arange(T)[:, None]
    lag = (1 << np.arange(L))[None, :]
    return ((t >= lag) & (lag < T)).astype(np.float64)


def tree_mask(ids, L, eot):
    """(B, T, L) level mask x doc-reset mask. doc(t) = number of EOTs strictly before t; the
    level-l edge into t is allowed iff doc(t) == doc((t - 2^l) mod T)."""
    ids = np.asarray(ids)
    B, T = ids.shape
    is_eot = (ids == eot).astype(np.int64)
    doc = np.cumsum(is_eot, axis=1) - is_eot
    t = np.arange(T)
    same = np.stack([doc == doc[:, (t - (1 << l)) % T] for l in range(L)], axis=-1)
    return level_mask(T, L)[None] * same.astype(np.float64)


def active_levels(L, T):
    """min(L, floor(log2 T) + 1), reference modeling_dispatcher.py:76."""
    return min(L, int(np.floor(np.log2(T))) + 1)


def gate_preacts(A, B, Wi, Wf, Wr, bi, bf, br, n_lv, mask=None):
    """(pre_i, pre_f, pre_r), each (nb, T, n_lv, H) float64. A, B (nb, T, GH); W (L, H, GH);
    biases (L, H); mask (nb, T, >= n_lv) or None."""
    A, B = _f64(A), _f64(B)
    Wi, Wf, Wr, bi, bf, br = (_f64(x) for x in (Wi, Wf, Wr, bi, bf, br))
    nb, T, GH = A.shape
    L, H = Wi.shape[0], Wi.shape[1]
    m = None if mask is None else _f64(mask)
    mL = 0 if m is None else m.shape[-1]
    outs = [np.zeros((nb, T, n_lv, H)) for _ in range(3)]
    _load().dh_oracle_gate_preacts(_p(A), _p(B), _p(Wi), _p(Wf), _p(Wr), _p(bi), _p(bf), _p(br),
                                   _p(m), mL, _p(outs[0]), _p(outs[1]), _p(outs[2]),
                                   nb, T, GH, H, L, n_lv)
    return tuple(outs)


def level_scan(pre_i, pre_f, pre_r, V0, H, mask=None):
    """Scanned state (nb, T, H*hd) float64 from pre-activations (nb, T, n_lv, H) and V0."""
    pi, pf, pr, V0 = (_f64(x) for x in (pre_i, pre_f, pre_r, V0))
    nb, T, n_lv, _ = pi.shape
    d = V0.shape[-1]
    m = None if mask is None else _f64(mask)
    mL = 0 if m is None else m.shape[-1]
    V = np.zeros_like(V0)
    scratch = np.zeros_like(V0)
    _load().dh_oracle_level_scan(_p(pi), _p(pf), _p(pr), _p(m), mL, _p(V0), _p(V), _p(scratch),
                                 nb, T, H, d // H, n_lv)
    return V


def decode_step(A, B_hist, Wi, Wf, Wr, bi, bf, br, t, rg_hist, V_ring, V0):
    """One tree-layer decode step at position t. rg_hist (nb, Tmax, L, H) and V_ring (nb, S, d)
    must be C-contiguous float64 arrays; they are updated in place. Returns Y (nb, d)."""
    for name, a in (("rg_hist", rg_hist), ("V_ring", V_ring)):
        if a.dtype != np.float64 or not a.flags.c_contiguous:
            raise TypeError(f"{name} must be a C-contiguous float64 array")
    A, B_hist, V0 = _f64(A), _f64(B_hist), _f64(V0)
    Wi, Wf, Wr, bi, bf, br = (_f64(x) for x in (Wi, Wf, Wr, bi, bf, br))
    nb, Tmax, GH = B_hist.shape
    L, H = Wi.shape[0], Wi.shape[1]
    S, d = V_ring.shape[1], V_ring.shape[2]
    Y = np.zeros((nb, d))
    _load().dh_oracle_decode_step(_p(A), _p(B_hist), _p(Wi), _p(Wf), _p(Wr), _p(bi), _p(bf), _p(br),
                                  int(t), _p(rg_hist), _p(V_ring), _p(V0), _p(Y),
                                  nb, Tmax, S, GH, H, d // H, L)
    return Y
