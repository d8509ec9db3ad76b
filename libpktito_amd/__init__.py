"""libpktito's int8 product path on one MI355X: the Python side of the C ABI.

The reference's seam is a C table, ``pk_kernels`` (backend/kernels.h:242-278
in peterheb/libpktito), whose int8 entries are

    quantize(pk_act *a, const float *x, size_t xs)
    gemm_q8(float *out, size_t os, const int8_t *w, const float *ws,
            const float *bias, uint32_t rows, const pk_act *a, int add)

``libpkhip.so`` (include/pk_hip.h) computes both on the GPU with the
reference's bits. This module binds it with ctypes and mirrors the two
functions with the same names, argument meanings and edge behaviour, on numpy
arrays (the host-pointer drop-in) or on device tensors (the device-resident
path; torch is used only for device memory and streams). There is no CPU
path here: if libpkhip.so is missing or no gfx950 device answers, calls raise.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libpkhip.so")

PK_HIP_OK = 0
PK_HIP_EINVAL = 1
PK_HIP_ENODEV = 2
PK_HIP_ENOMEM = 3
PK_HIP_EDEVICE = 4
PK_HIP_ENOTUP = 5
PK_HIP_EROUND = 6
PK_HIP_ETIMEOUT = 7


class PkHipError(RuntimeError):
    """A pk_hip_* call returned an error code."""

    def __init__(self, code, msg):
        super().__init__(f"pk_hip error {code}: {msg}")
        self.code = code


class Act(ctypes.Structure):
    """pk_act (backend/kernels.h:41-45): q [T][n] int8, d [T][n/qb] fp32."""
    _fields_ = [("q", ctypes.c_void_p), ("d", ctypes.c_void_p),
                ("n", ctypes.c_uint32), ("qb", ctypes.c_uint32), ("T", ctypes.c_uint32)]


class Seg(ctypes.Structure):
    """pk_hip_seg: one segment of a grouped product."""
    _fields_ = [("out", ctypes.c_void_p), ("os", ctypes.c_size_t), ("a", Act)]


class Job(ctypes.Structure):
    """pk_hip_job: one product of a batch."""
    _fields_ = [("out", ctypes.c_void_p), ("os", ctypes.c_size_t), ("m", ctypes.c_void_p),
                ("r0", ctypes.c_uint32), ("rows", ctypes.c_uint32), ("ws", ctypes.c_void_p),
                ("bias", ctypes.c_void_p), ("a", Act), ("qp", ctypes.c_void_p), ("add", ctypes.c_int)]


DEC_MAX_LAYERS = 8


class Decoder(ctypes.Structure):
    """pk_hip_decoder: the prediction network and joint for the device search."""
    _fields_ = [("P", ctypes.c_uint32), ("L", ctypes.c_uint32), ("J", ctypes.c_uint32), ("V", ctypes.c_uint32),
                ("n_dur", ctypes.c_uint32), ("blank", ctypes.c_uint32), ("max_symbols", ctypes.c_uint32),
                ("dur", ctypes.c_int32 * 64), ("embed", ctypes.c_void_p),
                ("wx", ctypes.c_void_p * DEC_MAX_LAYERS), ("wh", ctypes.c_void_p * DEC_MAX_LAYERS),
                ("b", ctypes.c_void_p * DEC_MAX_LAYERS), ("jpred", ctypes.c_void_p), ("jout", ctypes.c_void_p),
                ("jpred_b", ctypes.c_void_p), ("jout_b", ctypes.c_void_p)]


_F32P = ctypes.c_void_p
LAYER_VECTORS = ("ff1_nw", "ff1_nb", "att_nw", "att_nb", "conv_nw", "conv_nb", "ff2_nw", "ff2_nb", "out_nw",
                 "out_nb")
LAYER_MATRICES = ("ff1_up", "ff1_down", "ff2_up", "ff2_down", "q", "k", "v", "pos", "o", "pw1", "pw2")


class LayerW(ctypes.Structure):
    """pk_hip_layer: one encoder layer's weights on the device (core/model.h:45-53)."""
    _fields_ = ([("D", ctypes.c_uint32), ("H", ctypes.c_uint32), ("F", ctypes.c_uint32), ("K", ctypes.c_uint32),
                 ("eps", ctypes.c_float)] + [(n, _F32P) for n in LAYER_VECTORS] +
                [(n, ctypes.c_void_p) for n in ("ff1_up", "ff1_down", "ff2_up", "ff2_down", "q", "k", "v", "pos",
                                                "o")] +
                [("bias_u", _F32P), ("bias_v", _F32P), ("pw1", ctypes.c_void_p), ("pw2", ctypes.c_void_p),
                 ("dw", _F32P), ("dw_b", _F32P)])


_lib = None

# every function include/pk_hip.h declares, with its ctypes signature
_SIGS = {
    "pk_hip_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "pk_hip_last_error": (ctypes.c_char_p, []),
    "pk_hip_last_kernel": (ctypes.c_char_p, []),
    "pk_hip_tilings": (ctypes.c_int, []),
    "pk_hip_force_tiling": (ctypes.c_int, [ctypes.c_int]),
    "pk_hip_force_split": (ctypes.c_int, [ctypes.c_int]),
    "pk_hip_force_search_resident": (ctypes.c_int, [ctypes.c_int]),
    "pk_hip_gemm_workspace": (ctypes.c_size_t, [ctypes.c_uint32]),
    "pk_hip_tiling_name": (ctypes.c_char_p, [ctypes.c_int]),
    "pk_hip_force_quantize": (ctypes.c_int, [ctypes.c_int]),
    "pk_hip_force_attention": (ctypes.c_int, [ctypes.c_int]),
    "pk_hip_init": (ctypes.c_int, []),
    "pk_hip_upload_q8": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32]),
    "pk_hip_release_q8": (ctypes.c_int, [ctypes.c_void_p]),
    "pk_hip_release_all": (None, []),
    "pk_hip_quantize": (ctypes.c_int, [ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_size_t]),
    "pk_hip_gemm_q8": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(Act), ctypes.c_int]),
    "pk_hip_q8_find": (ctypes.c_void_p, [ctypes.c_void_p]),
    "pk_hip_q8_scales": (ctypes.c_void_p, [ctypes.c_void_p]),
    "pk_hip_q8_rows": (ctypes.c_uint32, [ctypes.c_void_p]),
    "pk_hip_q8_cols": (ctypes.c_uint32, [ctypes.c_void_p]),
    "pk_hip_quantize_dev": (ctypes.c_int, [ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "pk_hip_gemm_q8_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_uint32,
                                          ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(Act),
                                          ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "pk_hip_packed_bytes": (ctypes.c_size_t, [ctypes.c_uint32, ctypes.c_uint32]),
    "pk_hip_quantize_packed_dev": (ctypes.c_int, [ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_size_t, ctypes.c_void_p]),
    "pk_hip_gemm_q8_packed_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_uint32,
                                                 ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_void_p]),
    "pk_hip_gemm_q8_ws_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_uint32,
                                             ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(Act),
                                             ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                             ctypes.c_void_p]),
    "pk_hip_gemm_q8_packed_ws_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                                    ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                                    ctypes.c_void_p, ctypes.POINTER(Act), ctypes.c_void_p,
                                                    ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                                    ctypes.c_void_p]),
    "pk_hip_gemm_q8_grouped_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(Seg),
                                                  ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p]),
    "pk_hip_gemm_q8_batch_dev": (ctypes.c_int, [ctypes.POINTER(Job), ctypes.c_uint32, ctypes.c_int,
                                                ctypes.c_void_p]),
    "pk_hip_normq_dev": (ctypes.c_int, [ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p]),
    "pk_hip_siluq_dev": (ctypes.c_int, [ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                        ctypes.c_void_p]),
    "pk_hip_dwq_dev": (ctypes.c_int, [ctypes.POINTER(Act), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]),
    "pk_hip_layernorm_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p]),
    "pk_hip_attention_workspace": (ctypes.c_size_t, [ctypes.c_uint32, ctypes.c_uint32]),
    "pk_hip_attention_dev": (ctypes.c_int, [ctypes.c_void_p] * 7 + [ctypes.c_uint32] * 3 +
                             [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "pk_hip_empty_dev": (ctypes.c_int, [ctypes.c_void_p]),
    "pk_hip_stream_read_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]),
    "pk_hip_mfma_rate_dev": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]),
    "pk_hip_attention_noalloc_dev": (ctypes.c_int, [ctypes.c_void_p] * 7 + [ctypes.c_uint32] * 3 + [ctypes.c_void_p]),
    "pk_hip_layer_workspace": (ctypes.c_size_t, [ctypes.POINTER(LayerW), ctypes.c_uint32, ctypes.c_uint32]),
    "pk_hip_gemv_dev": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_void_p]),
    "pk_hip_lstm_step_dev": (ctypes.c_int, [ctypes.c_void_p] * 7 + [ctypes.c_void_p]),
    "pk_hip_search_workspace": (ctypes.c_size_t, [ctypes.POINTER(Decoder), ctypes.c_uint32]),
    "pk_hip_search_dev": (ctypes.c_int, [ctypes.POINTER(Decoder), ctypes.c_void_p, ctypes.c_uint32,
                                         ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint32),
                                         ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_void_p]),
    "pk_hip_joint_dev": (ctypes.c_int, [ctypes.c_void_p] * 6 + [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]),
    "pk_hip_layer_dev": (ctypes.c_int, [ctypes.POINTER(LayerW), ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_size_t,
                                        ctypes.c_void_p]),
}


def lib():
    """The loaded libpkhip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run python -m libpktito_amd.build "
                               "(the int8 path has no CPU fallback)")
        # One HIP runtime a process: torch's wheel carries its own
        # libamdhip64.so.7. Loaded first, it is the one libpkhip.so binds to
        # (same soname); loaded after libpkhip.so had pulled in /opt/rocm's,
        # torch would start a second runtime that sees no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _check(code):
    if code != PK_HIP_OK:
        raise PkHipError(code, lib().pk_hip_last_error().decode(errors="replace"))


def init():
    """Open the device (pk_hip_init); raises PkHipError when none is usable."""
    _check(lib().pk_hip_init())


def last_kernel():
    """The kernel variant the calling thread launched last."""
    return lib().pk_hip_last_kernel().decode()


def tilings():
    """How many tilings the per-column product has (pk_hip_tilings)."""
    return lib().pk_hip_tilings()


def tiling_name(index):
    """The name of tiling `index` (pk_hip_tiling_name)."""
    return lib().pk_hip_tiling_name(index).decode()


def tiling_index(name):
    """The index of the tiling called `name`, or -1."""
    for i in range(tilings()):
        if tiling_name(i) == name:
            return i
    return -1


def force_tiling(index):
    """Force tiling `index` for every later launch (-1: automatic); returns
    the one forced before."""
    return lib().pk_hip_force_tiling(index)


def force_quantize(kind):
    """Force the packed quantize's kernel for every later launch (0 one wave
    a column, or a wave a 1024-input chunk of a wide column in blocks; 1 one
    workgroup a 16-column group; 2 one wave a whole column; -1 automatic);
    returns the one forced before."""
    return lib().pk_hip_force_quantize(kind)


def force_attention(valu):
    """The attention's score and PV products for every later launch: 0 on
    the matrix cores (the default), 1 as VALU fma chains; returns the one
    set before."""
    return lib().pk_hip_force_attention(int(valu))


def _ptr(a):
    return a.ctypes.data if a is not None else None


# ------------------------------------------------------------ the drop-in ---

def make_act(q, d, n, qb, T):
    """A pk_act over numpy arrays (or raw addresses)."""
    qp = q if isinstance(q, int) else _ptr(q)
    dp = d if isinstance(d, int) else _ptr(d)
    return Act(qp, dp, n, qb, T)


def quantize(a, x, xs):
    """pk_k_quantize (backend/kernels.h:47-58) on host arrays: x holds T
    columns of a.n floats, column t at x[t * xs:]; fills a.q and a.d."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    _check(lib().pk_hip_quantize(ctypes.byref(a), _ptr(x), xs))


def gemm_q8(out, os_, w, ws, bias, rows, a, add, w_offset=0, out_offset=0):
    """pk_k_gemm_q8 (backend/kernels.h:60-78) on host arrays. w is the whole
    uploaded PK_Q8 matrix's bytes and w_offset the byte offset of the call's
    first panel inside it (the reference's w + r0 * cols); ws and bias start
    at that panel's first row; out_offset is the float offset of the call's
    first output (out + r0)."""
    assert out.dtype == np.float32 and ws.dtype == np.float32
    wp = _ptr(w) + w_offset
    op = _ptr(out) + 4 * out_offset
    _check(lib().pk_hip_gemm_q8(op, os_, wp, _ptr(ws), _ptr(bias), rows, ctypes.byref(a), int(add)))


class Q8Matrix:
    """A PK_Q8 matrix uploaded to HBM, repacked once (the model-load step).
    Keeps its host arrays alive, since the registry is keyed on their address."""

    def __init__(self, q, s):
        assert q.dtype == np.int8 and s.dtype == np.float32
        rows = s.shape[0]
        cols = q.size // rows
        self.q, self.s, self.rows, self.cols = q, s, rows, cols
        _check(lib().pk_hip_upload_q8(_ptr(q), _ptr(s), rows, cols))
        self.handle = lib().pk_hip_q8_find(_ptr(q))

    @property
    def dev_scales(self):
        return lib().pk_hip_q8_scales(self.handle)

    def release(self):
        if self.handle:
            _check(lib().pk_hip_release_q8(_ptr(self.q)))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.release()


# ------------------------------------------------ the device-resident path ---

def _dptr(t):
    return t.data_ptr() if t is not None else None


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return stream


def quantize_dev(q, d, x, n, qb, T, xs, stream=None):
    """quantize on device tensors: x float32 (T rows at stride xs), q int8
    [T, n], d float32 [T, n / qb]."""
    a = Act(_dptr(q), _dptr(d), n, qb, T)
    _check(lib().pk_hip_quantize_dev(ctypes.byref(a), _dptr(x), xs, _stream(stream)))


def gemm_q8_dev(out, os_, m, r0, rows, ws, bias, q, d, n, qb, T, add, rmode=0, stream=None,
                ws_ptr=None, out_ptr=None, work=None):
    """gemm_q8 on device tensors against an uploaded Q8Matrix m, rows
    [r0, r0 + rows). ws (or ws_ptr) and bias start at row r0; out (or
    out_ptr) at the first output. With work (a zeroed uint8 tensor of
    gemm_workspace(rows) bytes), few-frame products split K over the
    workspace (pk_hip_gemm_q8_ws_dev)."""
    a = Act(_dptr(q), _dptr(d), n, qb, T)
    wsp = ws_ptr if ws_ptr is not None else _dptr(ws)
    op = out_ptr if out_ptr is not None else _dptr(out)
    if work is not None:
        _check(lib().pk_hip_gemm_q8_ws_dev(op, os_, m.handle, r0, rows, wsp, _dptr(bias), ctypes.byref(a),
                                           int(add), rmode, _dptr(work), work.numel(), _stream(stream)))
        return
    _check(lib().pk_hip_gemm_q8_dev(op, os_, m.handle, r0, rows, wsp, _dptr(bias),
                                    ctypes.byref(a), int(add), rmode, _stream(stream)))


def gemm_workspace(rows):
    """Bytes of workspace a split few-frame product of rows channels takes
    (pk_hip_gemm_workspace)."""
    return lib().pk_hip_gemm_workspace(rows)


def force_split(splits):
    """Force how many workgroups share a panel in split few-frame products
    (1..8, -1 automatic); returns the one forced before."""
    return lib().pk_hip_force_split(splits)


def force_search_resident(on):
    """Whether later searches keep their panels resident where they fit
    (the default) or load them each token; returns the previous setting."""
    return bool(lib().pk_hip_force_search_resident(1 if on else 0))


def packed_bytes(n, T):
    """Bytes a packed copy of T columns of n inputs takes."""
    return lib().pk_hip_packed_bytes(n, T)


def quantize_packed_dev(q, qp, d, x, n, T, xs, stream=None, qb=None):
    """Quantize on device tensors into the packed copy qp (uint8/int8,
    packed_bytes(n, T) long), and into q [T, n] unless q is None; blocks of
    qb inputs (the whole row by default; 32 or 64)."""
    a = Act(_dptr(q), _dptr(d), n, qb or n, T)
    _check(lib().pk_hip_quantize_packed_dev(ctypes.byref(a), _dptr(qp), _dptr(x), xs, _stream(stream)))


def gemm_q8_packed_dev(out, os_, m, r0, rows, ws_ptr, bias, qp, d, n, T, add, rmode=0, stream=None, out_ptr=None,
                       qb=None, work=None):
    """gemm_q8 on device tensors with the activations from the packed copy qp
    (blocks of qb inputs: the whole row by default, or 32 or 64); work as for
    gemm_q8_dev (pk_hip_gemm_q8_packed_ws_dev)."""
    a = Act(None, _dptr(d), n, qb or n, T)
    op = out_ptr if out_ptr is not None else _dptr(out)
    if work is not None:
        _check(lib().pk_hip_gemm_q8_packed_ws_dev(op, os_, m.handle, r0, rows, ws_ptr, _dptr(bias),
                                                  ctypes.byref(a), _dptr(qp), int(add), rmode, _dptr(work),
                                                  work.numel(), _stream(stream)))
        return
    _check(lib().pk_hip_gemm_q8_packed_dev(op, os_, m.handle, r0, rows, ws_ptr, _dptr(bias), ctypes.byref(a),
                                           _dptr(qp), int(add), rmode, _stream(stream)))


def gemm_q8_grouped_dev(m, r0, rows, ws_ptr, bias, segs, add, stream=None):
    """One launch over segments [(out, os, q, d, n, qb, T), ...] of device tensors."""
    arr = (Seg * len(segs))()
    for i, (out, os_, q, d, n, qb, T) in enumerate(segs):
        arr[i] = Seg(_dptr(out), os_, Act(_dptr(q), _dptr(d), n, qb, T))
    _check(lib().pk_hip_gemm_q8_grouped_dev(m.handle, r0, rows, ws_ptr, _dptr(bias), arr, len(segs),
                                            int(add), _stream(stream)))


def gemm_q8_batch_dev(jobs, rmode=0, stream=None, qb=None):
    """Independent products in one launch: jobs [(out, os, m, r0, rows, ws_ptr,
    bias, qp, d, n, T, add), ...] of device tensors, m a Q8Matrix, qp packed
    activations in blocks of qb (default: per-row, qb = n)."""
    arr = (Job * len(jobs))()
    for i, (out, os_, m, r0, rows, ws_ptr, bias, qp, d, n, T, add) in enumerate(jobs):
        arr[i] = Job(_dptr(out), os_, m.handle, r0, rows, ws_ptr, _dptr(bias),
                     Act(None, _dptr(d), n, n if qb is None else qb, T), _dptr(qp), int(add))
    _check(lib().pk_hip_gemm_q8_batch_dev(arr, len(jobs), int(rmode), _stream(stream)))


# ----------------------------------------------- the device-resident layer ---

def normq_dev(qp, d, x, n, qb, T, w, b, eps, stream=None):
    """normq (core/encoder.c:108-128) on device tensors: T frames of n at x,
    layer-normed by w, b, eps, quantized in blocks of qb into qp and d."""
    a = Act(None, _dptr(d), n, qb, T)
    _check(lib().pk_hip_normq_dev(ctypes.byref(a), _dptr(qp), _dptr(x), _dptr(w), _dptr(b), eps, _stream(stream)))


def siluq_dev(qp, d, x, n, qb, T, xs, stream=None):
    """SiLU then the quantize (core/encoder.c:130-156) on device tensors."""
    a = Act(None, _dptr(d), n, qb, T)
    _check(lib().pk_hip_siluq_dev(ctypes.byref(a), _dptr(qp), _dptr(x), xs, _stream(stream)))


def dwq_dev(qp, d, u, n, qb, T, w, b, K, stream=None):
    """GLU of u [T, 2n], the depthwise convolution w [n, K] + b with SiLU,
    quantized (core/encoder.c:158-176)."""
    a = Act(None, _dptr(d), n, qb, T)
    _check(lib().pk_hip_dwq_dev(ctypes.byref(a), _dptr(qp), _dptr(u), _dptr(w), _dptr(b), K, _stream(stream)))


def layernorm_dev(x, T, n, w, b, eps, stream=None):
    """The layer norm in place over T rows of n floats."""
    _check(lib().pk_hip_layernorm_dev(_dptr(x), T, n, _dptr(w), _dptr(b), eps, _stream(stream)))


def attention_workspace(T, H):
    return lib().pk_hip_attention_workspace(T, H)


def attention_dev(o, q, k, v, p, bias_u, bias_v, T, D, H, ws, stream=None):
    """The attention's float part (core/encoder.c:280-327) on device tensors;
    ws a uint8 tensor of attention_workspace(T, H) bytes."""
    _check(lib().pk_hip_attention_dev(_dptr(o), _dptr(q), _dptr(k), _dptr(v), _dptr(p), _dptr(bias_u),
                                      _dptr(bias_v), T, D, H, _dptr(ws), ws.numel(), _stream(stream)))


def attention_noalloc_dev(o, q, k, v, p, bias_u, bias_v, T, D, H, stream=None):
    """attention_dev with the scores in the library's static scratch: no
    workspace, nothing allocated (pk_hip_attention_noalloc_dev)."""
    _check(lib().pk_hip_attention_noalloc_dev(_dptr(o), _dptr(q), _dptr(k), _dptr(v), _dptr(p), _dptr(bias_u),
                                              _dptr(bias_v), T, D, H, _stream(stream)))


def empty_dev(stream=None):
    """An empty kernel launch (the launch floor, for measurements)."""
    _check(lib().pk_hip_empty_dev(_stream(stream)))


def stream_read_dev(buf, sink, nbytes=None, stream=None):
    """A streaming read of nbytes (all of buf by default) of the device tensor
    buf, sink a device tensor of at least 4 bytes (the read floor, for
    measurements)."""
    n = buf.numel() * buf.element_size() if nbytes is None else nbytes
    _check(lib().pk_hip_stream_read_dev(_dptr(buf), n, _dptr(sink), _stream(stream)))


def mfma_rate_dev(workgroups, iters, sink, stream=None):
    """workgroups x 4 waves x iters x 8 int8 16x16x64 MFMAs (32768 ops each)
    on registers: the matrix cores' rate, for measurements."""
    _check(lib().pk_hip_mfma_rate_dev(workgroups, iters, _dptr(sink), _stream(stream)))


class DeviceLayer:
    """One encoder layer's weights in HBM: the eleven matrices uploaded
    (Q8Matrix), the vectors as device tensors. weights is a dict of numpy
    arrays: each of LAYER_VECTORS, bias_u, bias_v, dw [D, K], dw_b, and for
    each of LAYER_MATRICES the PK_Q8 bytes `name` and row scales `name_s`;
    and the shapes D, H, F, K and eps."""

    def __init__(self, weights, torch):
        dev = torch.device("cuda")
        self.D, self.H, self.F, self.K = (int(weights[k]) for k in ("D", "H", "F", "K"))
        self.st = LayerW(D=self.D, H=self.H, F=self.F, K=self.K, eps=float(weights["eps"]))
        self.tensors = {}
        for n in LAYER_VECTORS + ("bias_u", "bias_v", "dw", "dw_b"):
            t = torch.from_numpy(np.ascontiguousarray(weights[n], dtype=np.float32)).to(dev)
            self.tensors[n] = t
            setattr(self.st, n, t.data_ptr())
        self.mats = {}
        for n in LAYER_MATRICES:
            m = Q8Matrix(np.ascontiguousarray(weights[n], dtype=np.int8),
                         np.ascontiguousarray(weights[n + "_s"], dtype=np.float32))
            self.mats[n] = m
            setattr(self.st, n, m.handle)

    def workspace(self, T, qb):
        return lib().pk_hip_layer_workspace(ctypes.byref(self.st), T, qb)

    def run(self, x, T, ape_qp, ape_d, qb, ws, stream=None):
        """One layer in place on the device tensor x [T, D]; ws a uint8 tensor
        of at least workspace(T, qb) bytes."""
        _check(lib().pk_hip_layer_dev(ctypes.byref(self.st), _dptr(x), T, _dptr(ape_qp), _dptr(ape_d), qb,
                                      _dptr(ws), ws.numel(), _stream(stream)))

    def release(self):
        for m in self.mats.values():
            m.release()
        self.mats = {}


# ------------------------------------------------- the decoder's token steps ---

def gemv_dev(out, m, bias, x, add=0, stream=None):
    """gemv (core/decoder.c:54-63) on device tensors: x quantized whole, out[r]
    for every row of the uploaded m."""
    _check(lib().pk_hip_gemv_dev(_dptr(out), m.handle, _dptr(bias), _dptr(x), int(add), _stream(stream)))


def lstm_step_dev(h_out, c, h_in, x, wx, wh, b, stream=None, x_ptr=None):
    """One LSTM layer's step (core/decoder.c:68-75) on device tensors; x_ptr
    overrides x (a row of a device embedding)."""
    _check(lib().pk_hip_lstm_step_dev(_dptr(h_out), _dptr(c), _dptr(h_in), x_ptr if x_ptr is not None else _dptr(x),
                                      wx.handle, wh.handle, _dptr(b), _stream(stream)))


def joint_dev(logit, tok_dur, jout, jout_b, f, gp, V, n_dur, stream=None, f_ptr=None):
    """The joint (core/decoder.c:81-101) on device tensors: logits and
    tok_dur (int32 [2]) = (token, duration index)."""
    _check(lib().pk_hip_joint_dev(_dptr(logit), _dptr(tok_dur), jout.handle, _dptr(jout_b),
                                  f_ptr if f_ptr is not None else _dptr(f), _dptr(gp), V, n_dur, _stream(stream)))


class DeviceDecoder:
    """The prediction network and joint in HBM (matrices uploaded, vectors as
    device tensors), from a dict as libpktito_amd.synth.decoder_weights makes;
    its state (h, c of each layer, two h buffers a layer) stepped on device."""

    def __init__(self, dec, torch):
        self.torch = torch
        dev = torch.device("cuda")
        self.P, self.L, self.J, self.V, self.n_dur = (int(dec[k]) for k in ("P", "L", "J", "V", "n_dur"))
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
        self.embed = f32(dec["embed"])
        self.m = {}
        for n in [f"wx{l}" for l in range(self.L)] + [f"wh{l}" for l in range(self.L)] + ["jpred", "jout"]:
            self.m[n] = Q8Matrix(np.ascontiguousarray(dec[n], dtype=np.int8),
                                 np.ascontiguousarray(dec[n + "_s"], dtype=np.float32))
        self.b = [f32(dec[f"b{l}"]) for l in range(self.L)]
        self.jpred_b, self.jout_b = f32(dec["jpred_b"]), f32(dec["jout_b"])
        self.h = [[torch.zeros(self.P, dtype=torch.float32, device=dev) for _ in range(2)] for _ in range(self.L)]
        self.c = [torch.zeros(self.P, dtype=torch.float32, device=dev) for _ in range(self.L)]
        self.cur = [0] * self.L
        self.gp = torch.zeros(self.J, dtype=torch.float32, device=dev)
        self.logit = torch.zeros(self.m["jout"].rows, dtype=torch.float32, device=dev)
        self.tok_dur = torch.zeros(2, dtype=torch.int32, device=dev)

    def state(self):
        """(h [L, P], c [L, P]) as the layers hold them now."""
        h = self.torch.stack([self.h[l][self.cur[l]] for l in range(self.L)])
        return h, self.torch.stack(self.c)

    def set_state(self, h, c):
        for l in range(self.L):
            self.h[l][self.cur[l]].copy_(h[l])
            self.c[l].copy_(c[l])

    def predict(self, label, stream=None):
        """core/decoder.c:65-79: the label's embedding through the layers, then
        gp: L + 1 launches."""
        x_ptr = self.embed.data_ptr() + 4 * label * self.P
        for l in range(self.L):
            hin, hout = self.h[l][self.cur[l]], self.h[l][1 - self.cur[l]]
            lstm_step_dev(hout, self.c[l], hin, None, self.m[f"wx{l}"], self.m[f"wh{l}"], self.b[l], stream,
                          x_ptr=x_ptr)
            self.cur[l] = 1 - self.cur[l]
            x_ptr = hout.data_ptr()
        gemv_dev(self.gp, self.m["jpred"], self.jpred_b, self.h[self.L - 1][self.cur[self.L - 1]], 0, stream)

    def joint(self, f, stream=None, f_ptr=None):
        """core/decoder.c:81-101 at the frame whose encoder half is f."""
        joint_dev(self.logit, self.tok_dur, self.m["jout"], self.jout_b, f, self.gp, self.V, self.n_dur, stream,
                  f_ptr=f_ptr)

    def search(self, f, T, blank, durs, max_symbols, spin_limit=0, stream=None, f_ptr=None):
        """TDT's greedy search over T frames of the joint's encoder half f
        (device [T, J]) in one launch (pk_hip_search_dev): the tokens as
        (id, frame, duration). The state starts from zero, as the
        reference's pk_decode starts a segment."""
        d = Decoder()
        d.P, d.L, d.J, d.V, d.n_dur = self.P, self.L, self.J, self.V, self.n_dur
        d.blank, d.max_symbols = blank, max_symbols
        for i, v in enumerate(durs):
            d.dur[i] = int(v)
        d.embed = self.embed.data_ptr()
        for l in range(self.L):
            d.wx[l] = self.m[f"wx{l}"].handle
            d.wh[l] = self.m[f"wh{l}"].handle
            d.b[l] = self.b[l].data_ptr()
        d.jpred, d.jout = self.m["jpred"].handle, self.m["jout"].handle
        d.jpred_b, d.jout_b = self.jpred_b.data_ptr(), self.jout_b.data_ptr()
        cap = max(1, T * max_symbols)
        nbytes = lib().pk_hip_search_workspace(ctypes.byref(d), cap)
        if nbytes == 0:
            raise PkHipError(PK_HIP_EINVAL, "search: shapes the device search does not take")
        ws = self.torch.empty((nbytes + 256,), dtype=self.torch.uint8, device="cuda")
        wp = (ws.data_ptr() + 255) // 256 * 256
        toks = (ctypes.c_int32 * (3 * cap))()
        n = ctypes.c_uint32(0)
        fp = f_ptr if f_ptr is not None else _dptr(f)
        _check(lib().pk_hip_search_dev(ctypes.byref(d), fp, T, toks, cap, ctypes.byref(n), wp, nbytes, spin_limit,
                                       _stream(stream)))
        return [(toks[3 * i], toks[3 * i + 1], toks[3 * i + 2]) for i in range(n.value)]

    def release(self):
        for m in self.m.values():
            m.release()
        self.m = {}
