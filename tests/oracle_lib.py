"""ctypes handles on the oracle (oracle/liboracle.so, the CPU restatement) and,
where it was built, the reference's own compiled backends (oracle/_ref/
libpkref.so). Test infrastructure: what the tests compare against, never the
thing measured."""
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

_P, _Z, _U, _F, _I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_float, ctypes.c_int


def _float_sigs(l, pre, first):
    """argtypes of the float kernels, under prefix pre, with the extra leading
    arguments `first` (the backend index for the reference's)."""
    getattr(l, pre + "expf_n").argtypes = [_P, _P, _Z]
    getattr(l, pre + "sigmoidf_n").argtypes = [_P, _P, _Z]
    getattr(l, pre + "gemm_f32").argtypes = first + [_P, _Z, _P, _U, _U, _U, _P, _Z, _U, _P, _Z, _I]
    getattr(l, pre + "layernorm").argtypes = first + [_P, _Z, _P, _Z, _U, _U, _P, _P, _F]
    getattr(l, pre + "softmax").argtypes = first + [_P, _U, _F]
    getattr(l, pre + "silu").argtypes = first + [_P, _Z]
    getattr(l, pre + "glu").argtypes = first + [_P, _Z, _P, _Z, _U, _U]
    getattr(l, pre + "dwconv").argtypes = first + [_P, _Z, _P, _Z, _U, _U, _P, _P, _U]
    getattr(l, pre + "tanhf_n").argtypes = [_P, _P, _Z]
    getattr(l, pre + "lstm").argtypes = first + [_P, _P, _P, _U]


class Kernels(ctypes.Structure):
    """pko_kernels: the calls a layer makes, as function pointers."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("quantize", "gemm_q8", "gemm_f32", "layernorm", "softmax", "silu",
                                               "glu", "dwconv", "lstm")]


class Q8(ctypes.Structure):
    _fields_ = [("q", ctypes.c_void_p), ("s", ctypes.c_void_p), ("rows", ctypes.c_uint32),
                ("cols", ctypes.c_uint32)]


LAYER_NORMS = ("ff1_nw", "ff1_nb", "att_nw", "att_nb", "conv_nw", "conv_nb", "ff2_nw", "ff2_nb", "out_nw",
               "out_nb")
LAYER_MATS = ("ff1_up", "ff1_down", "ff2_up", "ff2_down", "q", "k", "v", "pos", "o", "pw1", "pw2")


class LstmW(ctypes.Structure):
    _fields_ = [("wx", Q8), ("wh", Q8), ("b", ctypes.c_void_p)]


class Decoder(ctypes.Structure):
    _fields_ = [("P", _U), ("L", _U), ("J", _U), ("V", _U), ("n_dur", _U), ("embed", ctypes.c_void_p),
                ("lstm", ctypes.POINTER(LstmW)), ("jpred", Q8), ("jpred_b", ctypes.c_void_p), ("jout", Q8),
                ("jout_b", ctypes.c_void_p)]


class Layer(ctypes.Structure):
    _fields_ = ([("D", ctypes.c_uint32), ("H", ctypes.c_uint32), ("F", ctypes.c_uint32), ("K", ctypes.c_uint32),
                 ("eps", ctypes.c_float)] + [(n, ctypes.c_void_p) for n in LAYER_NORMS] +
                [(n, Q8) for n in ("ff1_up", "ff1_down", "ff2_up", "ff2_down", "q", "k", "v", "pos", "o")] +
                [("bias_u", ctypes.c_void_p), ("bias_v", ctypes.c_void_p), ("pw1", Q8), ("pw2", Q8),
                 ("dw", ctypes.c_void_p), ("dw_b", ctypes.c_void_p)])


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
        _float_sigs(l, "pko_", [])
        l.pko_conformer_layer.argtypes = [ctypes.POINTER(Layer), ctypes.c_void_p, ctypes.c_uint32,
                                          ctypes.POINTER(Act), ctypes.c_uint32, ctypes.c_int]
        l.pko_conformer_layer_with.argtypes = [ctypes.POINTER(Kernels), ctypes.POINTER(Layer), ctypes.c_void_p,
                                               ctypes.c_uint32, ctypes.POINTER(Act), ctypes.c_uint32, ctypes.c_int]
        l.pko_predict_with.argtypes = [ctypes.POINTER(Kernels), ctypes.POINTER(Decoder), _U, _P, _P, _P, _P, _P]
        l.pko_joint_with.argtypes = [ctypes.POINTER(Kernels), ctypes.POINTER(Decoder), _P, _P, _P, _P, _P,
                                     ctypes.POINTER(_U), ctypes.POINTER(_U)]
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
        _float_sigs(l, "pkref_", [ctypes.c_int])
        l.pkref_kernels.argtypes = [ctypes.c_int, ctypes.POINTER(Kernels)]
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


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def expf(x, impl="oracle"):
    """core/vmath.h's pk_expf over an array, by the oracle or the reference."""
    x = _f32(x)
    y = np.empty_like(x)
    (oracle().pko_expf_n if impl == "oracle" else ref().pkref_expf_n)(_p(y), _p(x), x.size)
    return y


def sigmoidf(x, impl="oracle"):
    x = _f32(x)
    y = np.empty_like(x)
    (oracle().pko_sigmoidf_n if impl == "oracle" else ref().pkref_sigmoidf_n)(_p(y), _p(x), x.size)
    return y


def _float_call(name, impl, *args):
    if impl == "oracle":
        return getattr(oracle(), "pko_" + name)(*args)
    return getattr(ref(), "pkref_" + name)(ref_index(impl), *args)


def layernorm(x, w, b, eps, impl="oracle"):
    """pk_k_layernorm over the rows of x [T, n] into a new array."""
    x = _f32(x)
    T, n = x.shape
    out = np.empty_like(x)
    _float_call("layernorm", impl, _p(out), n, _p(x), n, T, n, _p(_f32(w)), _p(_f32(b)), eps)
    return out


def softmax(x, scale, impl="oracle"):
    """pk_k_softmax of each row of x [R, n], into a new array."""
    x = _f32(x).copy()
    for r in range(x.shape[0]):
        _float_call("softmax", impl, x[r].ctypes.data, x.shape[1], scale)
    return x


def silu(x, impl="oracle"):
    x = _f32(x).copy()
    _float_call("silu", impl, _p(x), x.size)
    return x


def glu(x, impl="oracle"):
    """pk_k_glu of x [T, 2n] into [T, n]."""
    x = _f32(x)
    T, n2 = x.shape
    out = np.empty((T, n2 // 2), np.float32)
    _float_call("glu", impl, _p(out), n2 // 2, _p(x), n2, T, n2 // 2)
    return out


def dwconv(x, w, b, impl="oracle"):
    """pk_k_dwconv of x [T, C] with taps w [C, K] and bias b [C]."""
    x = _f32(x)
    T, C = x.shape
    w = _f32(w)
    out = np.empty_like(x)
    _float_call("dwconv", impl, _p(out), C, _p(x), C, T, C, _p(w), _p(_f32(b)), w.shape[1])
    return out


def gemm_f32(w_panels, ld, rows, n, x, T, bias=None, bs=0, relu=0, impl="oracle"):
    """pk_k_gemm_f32 with its panel layout; out [T, rows]."""
    x = _f32(x)
    out = np.empty((T, rows), np.float32)
    _float_call("gemm_f32", impl, _p(out), rows, _p(_f32(w_panels)), ld, rows, n, _p(x), x.shape[1] if x.ndim > 1
                else n, T, _p(_f32(bias)) if bias is not None else None, bs, relu)
    return out


def conformer_layer(weights, x, T, ape_q, ape_d, qb, threads=8, impl="oracle"):
    """pko_conformer_layer on a copy of x [T, D]; weights is a dict of numpy
    arrays (LAYER_NORMS, bias_u, bias_v, dw, dw_b, and for each of LAYER_MATS
    the PK_Q8 panels `name` and row scales `name_s`) with the shapes D, H, F,
    K and eps. Returns the new x. impl names a reference backend ("ref",
    "avx512-vnni") to compose the layer from its kernels instead."""
    L = Layer(D=weights["D"], H=weights["H"], F=weights["F"], K=weights["K"], eps=weights["eps"])
    keep = []
    for n in LAYER_NORMS + ("bias_u", "bias_v", "dw", "dw_b"):
        a = _f32(weights[n])
        keep.append(a)
        setattr(L, n, a.ctypes.data)
    for n in LAYER_MATS:
        q = np.ascontiguousarray(weights[n], dtype=np.int8)
        s = _f32(weights[n + "_s"])
        keep += [q, s]
        setattr(L, n, Q8(q.ctypes.data, s.ctypes.data, s.size, q.size // s.size))
    y = _f32(x).copy()
    D = weights["D"]
    a = Act(_p(ape_q), _p(ape_d), D, qb, 2 * T - 1)
    if impl == "oracle":
        rc = oracle().pko_conformer_layer(ctypes.byref(L), _p(y), T, ctypes.byref(a), qb, threads)
    else:
        k = Kernels()
        ref().pkref_kernels(ref_index(impl), ctypes.byref(k))
        rc = oracle().pko_conformer_layer_with(ctypes.byref(k), ctypes.byref(L), _p(y), T, ctypes.byref(a), qb,
                                               threads)
    if rc:
        raise ValueError(f"pko_conformer_layer: {rc}")
    return y


def tanhf(x, impl="oracle"):
    """core/vmath.h's pk_tanhf over an array."""
    x = _f32(x)
    y = np.empty_like(x)
    (oracle().pko_tanhf_n if impl == "oracle" else ref().pkref_tanhf_n)(_p(y), _p(x), x.size)
    return y


def lstm(h, c, g, impl="oracle"):
    """pk_k_lstm: new (h, c) from copies of h, c [H] and the gates g [4H]."""
    h, c = _f32(h).copy(), _f32(c).copy()
    _float_call("lstm", impl, _p(h), _p(c), _p(_f32(g)), h.size)
    return h, c


def _kernels(impl):
    k = Kernels()
    if impl == "oracle":
        for n, _ in Kernels._fields_:
            setattr(k, n, ctypes.cast(getattr(oracle(), "pko_" + n), ctypes.c_void_p).value)
    else:
        ref().pkref_kernels(ref_index(impl), ctypes.byref(k))
    return k


class DecoderWeights:
    """The prediction network and joint in the oracle's structure: dec is a
    dict of numpy arrays (embed [V+1, P]; for each layer l wx{l}, wh{l} PK_Q8
    bytes with _s scales and b{l}; jpred, jout with _s and _b) and the shapes
    P, L, J, V, n_dur."""

    def __init__(self, dec):
        self.keep = []

        def q8(name):
            q = np.ascontiguousarray(dec[name], dtype=np.int8)
            s = _f32(dec[name + "_s"])
            self.keep += [q, s]
            return Q8(q.ctypes.data, s.ctypes.data, s.size, q.size // s.size)

        def vec(a):
            a = _f32(a)
            self.keep.append(a)
            return a.ctypes.data
        L = dec["L"]
        self.layers = (LstmW * L)()
        for l in range(L):
            self.layers[l] = LstmW(q8(f"wx{l}"), q8(f"wh{l}"), vec(dec[f"b{l}"]))
        self.st = Decoder(P=dec["P"], L=L, J=dec["J"], V=dec["V"], n_dur=dec["n_dur"], embed=vec(dec["embed"]),
                          lstm=self.layers, jpred=q8("jpred"), jpred_b=vec(dec["jpred_b"]), jout=q8("jout"),
                          jout_b=vec(dec["jout_b"]))
        self.P, self.L, self.J = dec["P"], L, dec["J"]
        self.rows = dec["jout_s"].size


def predict(dw, label, h, c, impl="oracle"):
    """core/decoder.c's predict: (new h [L, P], new c [L, P], gp [J])."""
    h, c = _f32(h).copy(), _f32(c).copy()
    gates = np.empty(4 * dw.P, np.float32)
    q = np.empty(max(dw.P, dw.J), np.int8)
    gp = np.empty(dw.J, np.float32)
    oracle().pko_predict_with(ctypes.byref(_kernels(impl)), ctypes.byref(dw.st), label, _p(h), _p(c), _p(gates),
                              _p(q), _p(gp))
    return h, c, gp


def joint(dw, f, gp, impl="oracle"):
    """core/decoder.c's joint: (logits, token, duration index)."""
    z = np.empty(dw.J, np.float32)
    q = np.empty(dw.J, np.int8)
    logit = np.empty(dw.rows, np.float32)
    tok, dur = _U(), _U()
    oracle().pko_joint_with(ctypes.byref(_kernels(impl)), ctypes.byref(dw.st), _p(_f32(f)), _p(_f32(gp)), _p(z),
                            _p(q), _p(logit), ctypes.byref(tok), ctypes.byref(dur))
    return logit, tok.value, dur.value
