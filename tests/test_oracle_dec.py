"""The oracle's decoder pieces, pinned on the CPU: tanh against the
reference's inline pk_tanhf and against tanh in double; the LSTM cell
against the reference's ref table; predict and joint (core/decoder.c:54-101)
against the same steps composed from the reference's own kernels and from its
avx512-vnni table; the argmax's first-of-equal rule on logits placed by hand
(zero joint weights make the logits exactly the bias)."""
import math

import numpy as np
import pytest

import oracle_lib as ol
from libpktito_amd import synth

needs_ref = pytest.mark.skipif(ol.ref() is None, reason="oracle/_ref not built (reference checkout absent)")


def bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return np.where(np.isnan(a), np.float32(np.nan), a).view(np.uint32)


@needs_ref
def test_tanh_is_the_references():
    g = synth.rng(1)
    x = np.concatenate([np.linspace(-12, 12, 200001, dtype=np.float32),
                        (g.standard_normal(100000) * 5).astype(np.float32),
                        np.array([0.625, -0.625, np.nextafter(np.float32(0.625), np.float32(0)), np.nan, np.inf,
                                  -np.inf, 0.0, -0.0, 1e-30, -1e-40], np.float32)])
    assert np.array_equal(bits(ol.tanhf(x)), bits(ol.tanhf(x, impl="ref")))


def test_tanh_is_close_to_tanh_in_double():
    # at most one float step from tanh in double rounded once to float, the
    # bound core/vmath.h states (bit patterns mapped to integers in order)
    def ordered(a):
        i = np.ascontiguousarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)
    x = np.linspace(-10, 10, 100001, dtype=np.float32)
    y = ordered(ol.tanhf(x))
    want = ordered(np.tanh(x.astype(np.float64)).astype(np.float32))
    assert np.max(np.abs(y - want)) <= 1
    # tanh(-0) is +0 by the reference's formula: fmaf(x x^2, p, x) with x = -0
    # and p < 0 is (-0 p) + -0 = +0 + -0 = +0
    z = ol.tanhf(np.array([0.0, -0.0], np.float32))
    assert z[0] == 0 and math.copysign(1, z[0]) > 0 and math.copysign(1, z[1]) > 0


@needs_ref
def test_lstm_cell_is_the_references():
    g = synth.rng(2)
    H = 64
    gates = (g.standard_normal(4 * H) * 4).astype(np.float32)
    gates[:4] = [0.0, -0.0, 90.0, -90.0]
    h, c = g.standard_normal(H).astype(np.float32), (2 * g.standard_normal(H)).astype(np.float32)
    a = ol.lstm(h, c, gates)
    b = ol.lstm(h, c, gates, impl="ref")
    assert np.array_equal(bits(a[0]), bits(b[0])) and np.array_equal(bits(a[1]), bits(b[1]))


def small_decoder(seed, P=64, L=2, J=64, V=40, n_dur=5):
    return synth.decoder_weights(synth.rng(seed), P=P, L=L, J=J, V=V, n_dur=n_dur)


def composed_predict(dec, label, h, c, impl):
    """core/decoder.c:65-79 from a backend's quantize, gemm_q8 and lstm."""
    P, J = dec["P"], dec["J"]
    h, c = h.copy(), c.copy()

    def gemv(name, bias, x, out=None):
        rows = dec[name + "_s"].size
        cols = dec[name].size // rows
        q, d = ol.quantize(np.ascontiguousarray(x, np.float32), 1, cols, cols, cols, impl=impl)
        o = np.zeros(rows, np.float32) if out is None else out
        ol.gemm_q8(o, 0, dec[name], dec[name + "_s"], bias, rows, q, d, cols, cols, 1, int(out is not None),
                   impl=impl)
        return o
    x = dec["embed"][label]
    for l in range(dec["L"]):
        gates = gemv(f"wx{l}", dec[f"b{l}"], x)
        gemv(f"wh{l}", None, h[l], out=gates)
        h[l], c[l] = ol.lstm(h[l], c[l], gates, impl=impl)
        x = h[l]
    return h, c, gemv("jpred", dec["jpred_b"], x)


@needs_ref
@pytest.mark.parametrize("label", [0, 7, 40])
def test_predict_is_the_references_kernels_composed(label):
    dec = small_decoder(3)
    g = synth.rng(4)
    h = g.standard_normal((2, 64)).astype(np.float32)
    c = g.standard_normal((2, 64)).astype(np.float32)
    dw = ol.DecoderWeights(dec)
    got = ol.predict(dw, label, h, c)
    want = composed_predict(dec, label, h, c, "ref")
    for a, b in zip(got, want):
        assert np.array_equal(bits(a), bits(b))
    for impl in ("ref", "avx512-vnni"):
        if ol.ref_index(impl) >= 0 and ol.ref().pkref_usable(ol.ref_index(impl)):
            other = ol.predict(dw, label, h, c, impl=impl)
            for a, b in zip(got, other):
                assert np.array_equal(bits(a), bits(b))


@needs_ref
def test_joint_is_the_references_kernels_composed():
    dec = small_decoder(5)
    g = synth.rng(6)
    dw = ol.DecoderWeights(dec)
    for _ in range(8):
        f, gp = g.standard_normal((2, 64)).astype(np.float32)
        logit, tok, dur = ol.joint(dw, f, gp)
        z = np.maximum(f + gp, 0).astype(np.float32)
        q, d = ol.quantize(z, 1, 64, 64, 64, impl="ref")
        want = np.zeros(dw.rows, np.float32)
        ol.gemm_q8(want, 0, dec["jout"], dec["jout_s"], dec["jout_b"], dw.rows, q, d, 64, 64, 1, 0, impl="ref")
        assert np.array_equal(bits(logit), bits(want))
        V = dec["V"]
        assert tok == int(np.argmax(want[:V + 1])) and dur == int(np.argmax(want[V + 1:V + 1 + dec["n_dur"]]))


def test_argmax_takes_the_first_of_equal_values():
    """Logits placed by hand through the bias (zero joint weights): ties go
    to the first, +0 and -0 are equal, a NaN never wins except at index 0,
    where nothing beats it (core/decoder.c:90-98)."""
    dec = small_decoder(8)
    V, n_dur = dec["V"], dec["n_dur"]
    dec["jout"] = np.zeros_like(dec["jout"])
    f = np.zeros(64, np.float32)
    cases = []
    b = np.zeros(dec["jout_b"].size, np.float32)
    b[5] = b[9] = 3.0
    b[V + 1 + 2] = b[V + 1 + 4] = 1.0
    cases.append((b.copy(), 5, 2))
    b = np.zeros_like(b)
    b[0] = -0.0
    b[3] = 0.0                                    # equal to -0: the first stays
    b[V + 1:V + 1 + n_dur] = -1.0
    cases.append((b.copy(), 0, 0))
    b = np.full_like(b, -1.0)
    b[2] = np.nan
    b[7] = 0.5
    cases.append((b.copy(), 7, 0))
    b = np.full_like(b, -1.0)
    b[0] = np.nan
    b[7] = 0.5
    cases.append((b.copy(), 0, 0))
    for bias, tok, dur in cases:
        dec["jout_b"] = bias
        dw = ol.DecoderWeights(dec)
        _, t, d = ol.joint(dw, f, f)
        assert (t, d) == (tok, dur)
