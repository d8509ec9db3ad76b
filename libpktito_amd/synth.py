"""Synthetic inputs of the shapes and distributions the int8 path is measured
on, and the PK_Q8 packing they are stored in.

The reference's model file stores each int8 matrix in PK_Q8 panels
(core/pkf.h:28-41): q(r, k) at ((r/16)(cols/4) + k/4) 64 + (r%16) 4 + k%4.
pack_q8 / unpack_q8 convert a row-major matrix to and from that layout.

The workloads are one FastConformer layer's int8 products (d_model 1024,
8 heads, feed-forward 4096, the convolution module's pointwise 2048 before
its GLU): the shapes core/encoder.c:329-368 multiplies, with weights int8
uniform in [-127, 127], per-channel scales uniform in [1e-3, 1e-2], and
activations N(0, 1) (half-normal into the down projections, whose inputs
follow a SiLU or ReLU).
"""
import numpy as np

D_MODEL = 1024
FF = 4096
CONV = 2048


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def pack_q8(w):
    """Row-major int8 [rows, cols] -> PK_Q8 panel bytes (flat int8)."""
    rows, cols = w.shape
    assert rows % 16 == 0 and cols % 4 == 0
    return np.ascontiguousarray(
        w.reshape(rows // 16, 16, cols // 4, 4).transpose(0, 2, 1, 3)).reshape(-1)


def unpack_q8(p, rows, cols):
    """PK_Q8 panel bytes -> row-major int8 [rows, cols]."""
    return np.ascontiguousarray(
        p.reshape(rows // 16, cols // 4, 16, 4).transpose(0, 2, 1, 3)).reshape(rows, cols)


def weights(g, rows, cols):
    """int8 uniform in [-127, 127], row-major [rows, cols]."""
    return g.integers(-127, 128, size=(rows, cols), dtype=np.int8)


def scales(g, rows):
    """fp32 per-channel scales uniform in [1e-3, 1e-2]."""
    return g.uniform(1e-3, 1e-2, size=rows).astype(np.float32)


def activations(g, m, k, half=False):
    """fp32 N(0, 1) [m, k], or |N(0, 1)| for a down projection's input."""
    x = g.standard_normal(size=(m, k), dtype=np.float32)
    return np.abs(x) if half else x


def layer_products(m):
    """One FastConformer layer's int8 products at m frames:
    (name, frames, inputs, outputs, half-normal inputs, add to the residual).
    The positions' projection takes 2m - 1 rows (core/encoder.c:467-469)."""
    d, f, c = D_MODEL, FF, CONV
    return [
        ("ff1_up", m, d, f, False, False),
        ("ff1_down", m, f, d, True, True),
        ("q", m, d, d, False, False),
        ("k", m, d, d, False, False),
        ("v", m, d, d, False, False),
        ("pos", 2 * m - 1, d, d, False, False),
        ("o", m, d, d, False, True),
        ("pw1", m, d, c, False, False),
        ("pw2", m, d, d, False, True),
        ("ff2_up", m, d, f, False, False),
        ("ff2_down", m, f, d, True, True),
    ]


def layer_ops(m):
    """Integer operations (2 M K N) of one layer's products at m frames."""
    return sum(2 * mm * k * n for _, mm, k, n, _, _ in layer_products(m))


def ragged_lengths(seed=2024, count=8, lo=150, hi=750):
    """Frame counts of a ragged batch of segments of 12 to 60 seconds at 80 ms
    frames, drawn from a seed."""
    return [int(v) for v in rng(seed).integers(lo, hi + 1, size=count)]


# ------------------------------------------------ exact, portable generator --
# For fixtures that must regenerate bit for bit on any numpy: splitmix64 of a
# counter, integer arithmetic only.

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x):
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


class Counter:
    """A counter-based stream: draw i of stream `seed` is splitmix64(seed << 40 | i)."""

    def __init__(self, seed):
        self.base = np.uint64(seed) << np.uint64(40)
        self.i = 0

    def bits(self, n):
        idx = np.arange(self.i, self.i + n, dtype=np.uint64) | self.base
        self.i += n
        return splitmix64(idx)

    def int8(self, n, lo=-127, hi=127):
        return ((self.bits(n) % np.uint64(hi - lo + 1)).astype(np.int64) + lo).astype(np.int8)

    def uniform(self, n, lo=-1.0, hi=1.0):
        u = (self.bits(n) >> np.uint64(40)).astype(np.float64) / float(1 << 24)
        return (lo + (hi - lo) * u).astype(np.float32)

    def awkward(self, n, scale):
        """kcheck's value classes (tests/kcheck.c:51-60 in the reference): one in
        24 each +0, -0, a subnormal, -30 scale, scale / 2; else uniform."""
        cls = (self.bits(n) % np.uint64(24)).astype(np.int64)
        v = self.uniform(n) * np.float32(scale)
        v = np.where(cls == 0, np.float32(0.0), v)
        v = np.where(cls == 1, np.float32(-0.0), v)
        v = np.where(cls == 2, np.float32(1e-40), v)
        v = np.where(cls == 3, np.float32(-scale * 30.0), v)
        v = np.where(cls == 4, np.float32(scale * 0.5), v)
        return v.astype(np.float32)


LAYER_VECTORS = ("ff1_nw", "ff1_nb", "att_nw", "att_nb", "conv_nw", "conv_nb", "ff2_nw", "ff2_nb", "out_nw",
                 "out_nb")


def layer_weights(g, D, H, F, K, eps=1e-5):
    """Seeded random weights of one encoder layer (core/model.h:45-53) as a
    dict of numpy arrays: the norms' weights and biases, for each matrix its
    row-major int8 (`name_rm`), PK_Q8 bytes (`name`) and row scales
    (`name_s`, small enough that the residual stream stays O(1)), the
    attention's biases and the depthwise taps, and the shapes D, H, F, K,
    eps."""
    w = {"D": D, "H": H, "F": F, "K": K, "eps": eps}
    for n in LAYER_VECTORS:
        w[n] = (1.0 + 0.1 * g.standard_normal(D)) if n.endswith("nw") else 0.1 * g.standard_normal(D)
    shapes = {"ff1_up": (F, D), "ff1_down": (D, F), "ff2_up": (F, D), "ff2_down": (D, F), "q": (D, D),
              "k": (D, D), "v": (D, D), "pos": (D, D), "o": (D, D), "pw1": (2 * D, D), "pw2": (D, D)}
    for n, (rows, cols) in shapes.items():
        w[n + "_rm"] = weights(g, rows, cols)
        w[n] = pack_q8(w[n + "_rm"])
        w[n + "_s"] = (g.uniform(0.5, 1.5, rows) / (127.0 * np.sqrt(cols))).astype(np.float32)
    w["bias_u"] = 0.1 * g.standard_normal(D)
    w["bias_v"] = 0.1 * g.standard_normal(D)
    w["dw"] = 0.3 * g.standard_normal((D, K))
    w["dw_b"] = 0.1 * g.standard_normal(D)
    return {k: (v.astype(np.float32) if isinstance(v, np.ndarray) and v.dtype == np.float64 else v)
            for k, v in w.items()}


def decoder_weights(g, P=640, L=2, J=640, V=1024, n_dur=5):
    """Seeded random weights of the prediction network and joint
    (core/model.h:57-60, 124-131) as a dict of numpy arrays: the label
    embedding [V + 1, P]; for each LSTM layer l, wx{l} and wh{l} [4P, P] as
    PK_Q8 bytes with row scales (_s) and the summed biases b{l}; jpred [J, P]
    and jout [n_out_pad, J] with scales and biases, jout's rows past V + 1 +
    n_dur zero (the model pads them to 16); and the shapes."""
    n_out = V + 1 + n_dur
    n_pad = (n_out + 15) // 16 * 16
    d = {"P": P, "L": L, "J": J, "V": V, "n_dur": n_dur}
    d["embed"] = (0.5 * g.standard_normal((V + 1, P))).astype(np.float32)

    def mat(name, rows, cols, live=None):
        w = weights(g, rows, cols)
        if live is not None:
            w[live:] = 0
        d[name] = pack_q8(w)
        d[name + "_s"] = (g.uniform(0.5, 1.5, rows) / (127.0 * np.sqrt(cols))).astype(np.float32)
    for l in range(L):
        mat(f"wx{l}", 4 * P, P)
        mat(f"wh{l}", 4 * P, P)
        d[f"b{l}"] = (0.1 * g.standard_normal(4 * P)).astype(np.float32)
    mat("jpred", J, P)
    d["jpred_b"] = (0.1 * g.standard_normal(J)).astype(np.float32)
    mat("jout", n_pad, J, live=n_out)
    jb = (0.1 * g.standard_normal(n_pad)).astype(np.float32)
    jb[n_out:] = 0
    d["jout_b"] = jb
    return d
