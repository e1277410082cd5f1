"""ctypes bindings to the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only to check or time the reference's CPU algorithm. The product library never
uses it. Each wrapper names the flash.c lines its C function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")

TOL = 8e-3  # flash.c:935-937


def build(force=False):
    """Compile liboracle.so with the committed Makefile (gcc, -O2, no fast-math)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "liboracle.so"], cwd=_HERE,
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_bf16_n.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.orc_bf16_selfcheck.restype = ctypes.c_long
        L.orc_bf16_selfcheck.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        L.orc_lcg_bf16.argtypes = [ctypes.POINTER(ctypes.c_uint32), _u16p, ctypes.c_size_t]
        L.orc_normal_bf16.argtypes = [_u16p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64,
                                      ctypes.c_double]
        L.orc_attn_ref.restype = ctypes.c_int
        L.orc_attn_ref.argtypes = [_u16p, _u16p, _u16p, _f32p] + [ctypes.c_int] * 6 + [
            _i32p, ctypes.c_int]
        L.orc_attn_ref_mt.restype = ctypes.c_int
        L.orc_attn_ref_mt.argtypes = [_u16p, _u16p, _u16p, _f32p] + [ctypes.c_int] * 6 + [
            _i32p, ctypes.c_int, ctypes.c_int]
        L.orc_attn_pairs.restype = ctypes.c_double
        L.orc_attn_pairs.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_ref_rowset.restype = ctypes.c_int
        L.orc_ref_rowset.argtypes = [ctypes.c_int, ctypes.c_int, _i32p]
        L.orc_cmp_rows_tol.restype = ctypes.c_int
        L.orc_cmp_rows_tol.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       _i32p, ctypes.c_int, ctypes.c_float,
                                       ctypes.POINTER(ctypes.c_float),
                                       ctypes.POINTER(ctypes.c_float),
                                       ctypes.POINTER(ctypes.c_long)]
        _lib = L
    return _lib


# ---- bf16 helpers (flash.c:78-92) ---------------------------------------------------------
def f32_to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def bf16_selfcheck(lo=0, hi=0xFFFFFFFF):
    return lib().orc_bf16_selfcheck(lo, hi)


# ---- data modes ---------------------------------------------------------------------------
def lcg_qkv(Hq, Hkv, Sq, Sk, D, seed=0x12345678):
    """The reference's per-case data (flash.c:1030,1050-1061): Q, then K, then V."""
    st = ctypes.c_uint32(seed)
    Q = np.empty(Hq * Sq * D, np.uint16)
    K = np.empty(Hkv * Sk * D, np.uint16)
    V = np.empty(Hkv * Sk * D, np.uint16)
    for a in (Q, K, V):
        lib().orc_lcg_bf16(ctypes.byref(st), a, a.size)
    return Q, K, V


def normal_bf16(n, seed, counter0=0, sigma=1.0):
    out = np.empty(n, np.uint16)
    lib().orc_normal_bf16(out, n, seed, counter0, sigma)
    return out


def normal_qkv(Hq, Hkv, Sq, Sk, D, seed, sigma_q=1.0, sigma_kv=1.0):
    nq, nk = Hq * Sq * D, Hkv * Sk * D
    Q = normal_bf16(nq, seed, 0, sigma_q)
    K = normal_bf16(nk, seed, nq, sigma_kv)
    V = normal_bf16(nk, seed, nq + nk, sigma_kv)
    return Q, K, V


# ---- oracle, rows, compare ----------------------------------------------------------------
def ref_rowset(Sq, ref_cap):
    rows = np.empty(max(Sq, 1), np.int32)
    n = lib().orc_ref_rowset(Sq, ref_cap, rows)
    return rows[:n].copy()


def attn_ref(Q, K, V, Hq, Hkv, Sq, Sk, D, causal, rows=None, nthreads=1, out=None):
    """fp32 oracle (flash.c:262-314) over the listed rows; other rows stay zero."""
    if rows is None:
        rows = np.arange(Sq, dtype=np.int32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    O = out if out is not None else np.zeros(Hq * Sq * D, np.float32)
    # the C oracle indexes raw pointers: the arrays must hold the shapes they are said to have
    if (np.asarray(Q).size < Hq * Sq * D or np.asarray(K).size < Hkv * Sk * D or
            np.asarray(V).size < Hkv * Sk * D or O.size < Hq * Sq * D):
        raise ValueError("attn_ref: an array is smaller than its (H, S, D) shape")
    if rows.size and (rows.min() < 0 or rows.max() >= Sq):
        raise ValueError("attn_ref: a row index is outside [0, Sq)")
    if nthreads == 1:
        rc = lib().orc_attn_ref(Q, K, V, O, Hq, Hkv, Sq, Sk, D, int(causal), rows, rows.size)
    else:
        rc = lib().orc_attn_ref_mt(Q, K, V, O, Hq, Hkv, Sq, Sk, D, int(causal), rows, rows.size,
                                   nthreads)
    if rc != 0:
        raise ValueError("orc_attn_ref rejected the shape")
    return O


def attn_pairs(Sq, Sk, causal):
    return lib().orc_attn_pairs(Sq, Sk, int(causal))


def cmp_rows(Oref, Odut, Hq, Sq, D, rows, tol=TOL):
    """(ok, mad, maxref, nbad) per flash.c:939-980."""
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    mad, maxref, nbad = ctypes.c_float(), ctypes.c_float(), ctypes.c_long()
    ok = lib().orc_cmp_rows_tol(np.ascontiguousarray(Oref, np.float32).reshape(-1),
                                np.ascontiguousarray(Odut, np.float32).reshape(-1), Hq, Sq, D,
                                rows, rows.size, tol, ctypes.byref(mad), ctypes.byref(maxref),
                                ctypes.byref(nbad))
    return bool(ok), mad.value, maxref.value, nbad.value
