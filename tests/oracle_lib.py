"""ctypes handles on the oracle (oracle/liboracle.so, the CPU restatement) and,
where it was built, the reference's own compiled backends (oracle/_ref/
libpkref.so). Test infrastructure: the checker, never the thing measured."""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libpkref.so")


class Act(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("d", ctypes.c_void_p),
                ("n", ctypes.c_uint32), ("qb", ctypes.c_uint32), ("T", ctypes.c_uint32)]


_GEMM = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
         ctypes.c_uint32, ctypes.POINTER(Act), ctypes.c_int]

_oracle = None
_ref = None


def oracle():
    """liboracle.so, built with the oracle's Makefile if missing (gcc only)."""
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            subprocess.run(["make", "-s", "-C", ORACLE_DIR, "liboracle.so"], check=True)
        l = ctypes.CDLL(ORACLE_SO)
        l.pko_quantize.argtypes = [ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_size_t]
        l.pko_gemm_q8.argtypes = _GEMM
        l.pko_definition.argtypes = _GEMM[:-1]
        l.pko_fmaf.argtypes = [ctypes.c_float] * 3
        l.pko_fmaf.restype = ctypes.c_float
        l.pko_q8_index.argtypes = [ctypes.c_uint32] * 3
        l.pko_q8_index.restype = ctypes.c_size_t
        l.pko_gemm_threads.argtypes = [ctypes.c_void_p, ctypes.c_int] + _GEMM
        l.pko_quantize_threads.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(Act),
                                           ctypes.c_void_p, ctypes.c_size_t]
        _oracle = l
    return _oracle


def ref():
    """libpkref.so (the reference's ref and x86 backends) or None if not built."""
    global _ref
    if _ref is None and os.path.exists(REF_SO):
        l = ctypes.CDLL(REF_SO)
        l.pkref_id.restype = ctypes.c_char_p
        l.pkref_name.restype = ctypes.c_char_p
        l.pkref_quantize.argtypes = [ctypes.c_int, ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_size_t]
        l.pkref_gemm_q8.argtypes = [ctypes.c_int] + _GEMM
        l.pkref_gemm_threads.argtypes = [ctypes.c_int, ctypes.c_int] + _GEMM
        l.pkref_quantize_threads.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(Act),
                                             ctypes.c_void_p, ctypes.c_size_t]
        _ref = l
    return _ref


def ref_index(backend_id):
    """The libpkref.so index of a backend ("ref", "avx512-vnni", ...), or -1."""
    r = ref()
    if r is None:
        return -1
    for i in range(r.pkref_count()):
        if r.pkref_id(i).decode() == backend_id:
            return i
    return -1


def _p(a):
    return a.ctypes.data if a is not None else None


def quantize(x, T, n, qb, xs, impl="oracle"):
    """(q [T*n] int8, d [T*n/qb] float32) by the oracle, or by a reference
    backend when impl names one ("ref", "avx512-vnni")."""
    q = np.zeros(T * n, np.int8)
    d = np.zeros(T * (n // qb), np.float32)
    a = Act(_p(q), _p(d), n, qb, T)
    if impl == "oracle":
        oracle().pko_quantize(ctypes.byref(a), _p(x), xs)
    else:
        ref().pkref_quantize(ref_index(impl), ctypes.byref(a), _p(x), xs)
    return q, d


def gemm_q8(out, os_, w, ws, bias, rows, q, d, n, qb, T, add, impl="oracle", r0=0, threads=1):
    """out (float32, modified in place) by the oracle or a reference backend,
    for rows [r0, r0 + rows) of the PK_Q8 matrix w (whole-matrix bytes); the
    oracle over `threads` threads in 64-row slices when threads > 1."""
    a = Act(_p(q), _p(d), n, qb, T)
    wp = _p(w) + r0 * n
    op = _p(out) + 4 * r0
    wsp = _p(ws) + 4 * r0
    bp = _p(bias) + 4 * r0 if bias is not None else None
    if impl == "oracle" and threads > 1:
        fn = ctypes.cast(oracle().pko_gemm_q8, ctypes.c_void_p).value
        oracle().pko_gemm_threads(fn, threads, op, os_, wp, wsp, bp, rows, ctypes.byref(a), add)
    elif impl == "oracle":
        oracle().pko_gemm_q8(op, os_, wp, wsp, bp, rows, ctypes.byref(a), add)
    else:
        ref().pkref_gemm_q8(ref_index(impl), op, os_, wp, wsp, bp, rows, ctypes.byref(a), add)


def definition(w, ws, bias, rows, q, d, n, qb, T):
    """The int64 definition's outputs [T, rows] (no add)."""
    out = np.zeros(T * rows, np.float32)
    a = Act(_p(q), _p(d), n, qb, T)
    oracle().pko_definition(_p(out), rows, _p(w), _p(ws), _p(bias), rows, ctypes.byref(a))
    return out
