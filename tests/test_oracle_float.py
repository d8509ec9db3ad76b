"""The oracle's float kernels and its encoder layer, pinned on the CPU: each
kernel against the reference's own compiled ref table (oracle/_ref) on
seeded rows with NaNs, infinities, signed zeros, ties and the exp clamp's
ends; exp against exp in double; the layer norm against float64; and the
layer against a second composition of the reference's own kernels in
core/encoder.c's order, with layouts built here by numpy, and against what
the mathematics fixes (one frame's attention is its values)."""
import numpy as np
import pytest

import oracle_lib as ol
from layer_ref import attention, layer_weights, positions
from libpktito_amd import synth

needs_ref = pytest.mark.skipif(ol.ref() is None, reason="oracle/_ref not built (reference checkout absent)")


def bits(a):
    """The bit patterns, every NaN as one: which NaN an operation on
    non-finite inputs returns is the hardware's (x86 gives 0xffc00000 for
    inf - inf, gfx950 0x7fc00000), and the kernels' contract is on numbers,
    so NaNs compare as NaN and everything else to the bit."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    return np.where(np.isnan(a), np.float32(np.nan), a).view(np.uint32)


def awkward(g, shape, scale=4.0):
    """N(0, scale) with NaNs, infinities, signed zeros and values at the exp
    clamp's ends sprinkled in."""
    x = (g.standard_normal(shape) * scale).astype(np.float32)
    flat = x.reshape(-1)
    n = flat.size
    idx = g.integers(0, n, max(1, n // 50))
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 87.0, -87.0, 88.0, 88.5, -87.5, 1e-30, -1e-30,
                         0.5, -0.5], np.float32)
    flat[idx] = specials[g.integers(0, specials.size, idx.size)]
    return x


def test_expf_is_within_one_ulp_of_exp():
    # at most one float step from exp in double rounded once to float, the
    # bound core/vmath.h states for [-87, 88] (positive results: the bit
    # patterns order as the values do)
    x = np.linspace(-87.0, 88.0, 400001, dtype=np.float32)
    y = bits(ol.expf(x)).astype(np.int64)
    want = bits(np.exp(x.astype(np.float64)).astype(np.float32)).astype(np.int64)
    assert np.max(np.abs(y - want)) <= 1
    # the clamp: beyond it the ends' values; a NaN takes the low end's
    e = ol.expf(np.array([-200.0, -87.0, 88.0, 200.0, np.nan], np.float32))
    assert e[0] == e[1] and e[2] == e[3] and e[4] == e[0]


@needs_ref
def test_expf_and_sigmoid_are_the_references():
    g = synth.rng(11)
    x = np.concatenate([awkward(g, 200000, 30.0), np.linspace(-90, 90, 100001, dtype=np.float32)])
    assert np.array_equal(bits(ol.expf(x)), bits(ol.expf(x, impl="ref")))
    assert np.array_equal(bits(ol.sigmoidf(x)), bits(ol.sigmoidf(x, impl="ref")))


@needs_ref
@pytest.mark.parametrize("T,n", [(1, 16), (7, 1024), (33, 4096), (5, 80)])
def test_layernorm_is_the_references(T, n):
    g = synth.rng(T + n)
    x = awkward(g, (T, n))
    x[0] = g.standard_normal(n).astype(np.float32)    # one clean row at least
    w, b = g.standard_normal(n).astype(np.float32), g.standard_normal(n).astype(np.float32)
    assert np.array_equal(bits(ol.layernorm(x, w, b, 1e-5)), bits(ol.layernorm(x, w, b, 1e-5, impl="ref")))


def test_layernorm_is_close_to_float64():
    g = synth.rng(5)
    x = (g.standard_normal((40, 1024)) * 3 + 1).astype(np.float32)
    w, b = g.standard_normal(1024).astype(np.float32), g.standard_normal(1024).astype(np.float32)
    y = ol.layernorm(x, w, b, 1e-5)
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5) * w + b
    assert np.max(np.abs(y - want)) < 1e-4


@needs_ref
@pytest.mark.parametrize("n", [1, 16, 17, 750, 1499])
def test_softmax_is_the_references(n):
    g = synth.rng(n)
    x = awkward(g, (6, n), 8.0)
    x[0] = g.standard_normal(n).astype(np.float32)
    x[1] = 0.0
    x[1, n // 2] = -0.0
    scale = np.float32(1.0) / np.sqrt(np.float32(128.0))
    a, b = ol.softmax(x, scale), ol.softmax(x, scale, impl="ref")
    assert np.array_equal(bits(a), bits(b))
    assert abs(float(a[0].astype(np.float64).sum()) - 1.0) < 1e-5


@needs_ref
def test_silu_glu_dwconv_are_the_references():
    g = synth.rng(3)
    x = awkward(g, (37, 256))
    assert np.array_equal(bits(ol.silu(x)), bits(ol.silu(x, impl="ref")))
    assert np.array_equal(bits(ol.glu(x)), bits(ol.glu(x, impl="ref")))
    for T, K in ((37, 9), (3, 9), (20, 31), (1, 9)):
        h = awkward(g, (T, 128))
        w, b = g.standard_normal((128, K)).astype(np.float32), g.standard_normal(128).astype(np.float32)
        assert np.array_equal(bits(ol.dwconv(h, w, b)), bits(ol.dwconv(h, w, b, impl="ref")))


@needs_ref
@pytest.mark.parametrize("rows,n,T,ld", [(16, 128, 5, 128), (64, 750, 3, 752), (128, 64, 17, 80)])
def test_gemm_f32_is_the_references(rows, n, T, ld):
    g = synth.rng(rows + n)
    w = awkward(g, (rows // 16) * ld * 16, 1.0)
    x = awkward(g, (T, n), 1.0)
    bias = g.standard_normal(rows).astype(np.float32)
    for bb, relu in ((None, 0), (bias, 1)):
        a = ol.gemm_f32(w, ld, rows, n, x, T, bb, 0, relu)
        b = ol.gemm_f32(w, ld, rows, n, x, T, bb, 0, relu, impl="ref")
        assert np.array_equal(bits(a), bits(b))


# ------------------------------------------------------------- the layer --


def composed_layer(w, x, T, ape_q, ape_d, qb, impl):
    """core/encoder.c:321-368 composed here from a backend's kernels (the
    reference's ref table), the attention's panels laid out by numpy."""
    D, H, F, K, eps = w["D"], w["H"], w["F"], w["K"], w["eps"]
    dk = D // H
    x = x.copy()

    def gemm(mat, act_q, act_d, n, rows=None):
        rows = rows or w[mat + "_s"].size
        out = np.zeros(T * rows, np.float32)
        ol.gemm_q8(out, rows, w[mat], w[mat + "_s"], None, rows, act_q, act_d, n, qb, T, 0, impl=impl)
        return out.reshape(T, rows)

    def quant(v):
        return ol.quantize(np.ascontiguousarray(v, np.float32).reshape(-1), v.shape[0], v.shape[1], qb,
                           v.shape[1], impl=impl)

    def ff(nw, nb, up, down):
        aq, ad = quant(ol.layernorm(x, w[nw], w[nb], eps, impl=impl))
        hq, hd = quant(ol.silu(gemm(up, aq, ad, D), impl=impl))
        return gemm(down, hq, hd, F)

    x = x + ff("ff1_nw", "ff1_nb", "ff1_up", "ff1_down")
    aq, ad = quant(ol.layernorm(x, w["att_nw"], w["att_nb"], eps, impl=impl))
    q, k, v = gemm("q", aq, ad, D), gemm("k", aq, ad, D), gemm("v", aq, ad, D)
    R = 2 * T - 1
    pout = np.zeros(R * D, np.float32)
    ol.gemm_q8(pout, D, w["pos"], w["pos_s"], None, D, ape_q, ape_d, D, qb, R, 0, impl=impl)
    p = pout.reshape(R, D)
    o = attention(q, k, v, p, w["bias_u"], w["bias_v"], H, impl)
    aq, ad = quant(o)
    x = x + gemm("o", aq, ad, D)
    aq, ad = quant(ol.layernorm(x, w["conv_nw"], w["conv_nb"], eps, impl=impl))
    u = gemm("pw1", aq, ad, D)
    hh = ol.dwconv(ol.glu(u, impl=impl), w["dw"], w["dw_b"], impl=impl)
    aq, ad = quant(hh)
    x = x + gemm("pw2", aq, ad, D)
    x = x + ff("ff2_nw", "ff2_nb", "ff2_up", "ff2_down")
    return ol.layernorm(x, w["out_nw"], w["out_nb"], eps, impl=impl)


@needs_ref
@pytest.mark.parametrize("T,qb", [(37, 32), (16, 64), (1, 32), (2, 32)])
def test_layer_is_the_references_kernels_composed(T, qb):
    """The oracle's layer against the reference's ref kernels composed in
    core/encoder.c's order here. The residual adds here are the products'
    add = 1 (out + v, one rounding), the same bits."""
    g = synth.rng(T * 5 + qb)
    w = layer_weights(g, D=128, H=2, F=256, K=9)
    x = g.standard_normal((T, 128)).astype(np.float32)
    _, ape_q, ape_d = positions(g, T, 128, qb)
    got = ol.conformer_layer(w, x, T, ape_q, ape_d, qb, threads=4)
    want = composed_layer(w, x, T, ape_q, ape_d, qb, impl="ref")
    assert np.array_equal(bits(got), bits(want))


@needs_ref
@pytest.mark.parametrize("impl", ["ref", "avx512-vnni"])
def test_layer_from_the_references_table(impl):
    """The layer composed from a reference backend's own table (what the CPU
    baseline times) gives the oracle's bits."""
    if ol.ref_index(impl) < 0 or not ol.ref().pkref_usable(ol.ref_index(impl)):
        pytest.skip(f"{impl} not usable on this CPU")
    g = synth.rng(41)
    w = layer_weights(g, D=128, H=2, F=256, K=9)
    x = g.standard_normal((29, 128)).astype(np.float32)
    _, ape_q, ape_d = positions(g, 29, 128, 32)
    a = ol.conformer_layer(w, x, 29, ape_q, ape_d, 32, threads=3)
    b = ol.conformer_layer(w, x, 29, ape_q, ape_d, 32, threads=5, impl=impl)
    assert np.array_equal(bits(a), bits(b))


def test_layer_bits_do_not_depend_on_threads():
    g = synth.rng(99)
    w = layer_weights(g, D=128, H=2, F=256, K=9)
    x = g.standard_normal((23, 128)).astype(np.float32)
    _, ape_q, ape_d = positions(g, 23, 128, 32)
    a = ol.conformer_layer(w, x, 23, ape_q, ape_d, 32, threads=1)
    b = ol.conformer_layer(w, x, 23, ape_q, ape_d, 32, threads=7)
    assert np.array_equal(bits(a), bits(b)) and np.all(np.isfinite(a))


def test_layer_of_one_frame_attends_to_itself():
    """With one frame the softmax is over one key, e / e = 1 exactly, so the
    attention's output is its values: the oracle's layer equals the same
    layer with the attention replaced by v."""
    g = synth.rng(7)
    D = 128
    w = layer_weights(g, D=D, H=2, F=256, K=9)
    x = g.standard_normal((1, D)).astype(np.float32)
    _, ape_q, ape_d = positions(g, 1, D, 32)
    got = ol.conformer_layer(w, x, 1, ape_q, ape_d, 32, threads=1)
    # the same layer by hand with o = v (the oracle's own kernels)
    eps = w["eps"]

    def gemm(mat, aq, ad, n):
        rows = w[mat + "_s"].size
        out = np.zeros(rows, np.float32)
        ol.gemm_q8(out, rows, w[mat], w[mat + "_s"], None, rows, aq, ad, n, 32, 1, 0)
        return out.reshape(1, rows)

    def quant(v):
        return ol.quantize(np.ascontiguousarray(v, np.float32).reshape(-1), 1, v.shape[1], 32, v.shape[1])

    def ff(y, nw, nb, up, down):
        aq, ad = quant(ol.layernorm(y, w[nw], w[nb], eps))
        hq, hd = quant(ol.silu(gemm(up, aq, ad, D)))
        return y + gemm(down, hq, hd, 256)

    y = ff(x, "ff1_nw", "ff1_nb", "ff1_up", "ff1_down")
    aq, ad = quant(ol.layernorm(y, w["att_nw"], w["att_nb"], eps))
    o = gemm("v", aq, ad, D)
    aq, ad = quant(o)
    y = y + gemm("o", aq, ad, D)
    aq, ad = quant(ol.layernorm(y, w["conv_nw"], w["conv_nb"], eps))
    hh = ol.glu(gemm("pw1", aq, ad, D))
    # one frame: only the centre tap reads a frame
    K = w["K"]
    v = np.array([ol_fma(w["dw"][c, K // 2], hh[0, c]) + w["dw_b"][c] for c in range(D)], np.float32)[None]
    hh = v * ol.sigmoidf(v)
    aq, ad = quant(hh)
    y = y + gemm("pw2", aq, ad, D)
    y = ff(y, "ff2_nw", "ff2_nb", "ff2_up", "ff2_down")
    want = ol.layernorm(y, w["out_nw"], w["out_nb"], eps)
    assert np.array_equal(bits(got), bits(want))


def ol_fma(a, b):
    """fmaf(a, b, +0) = a * b rounded once: the product in double is exact."""
    return np.float32(np.float64(a) * np.float64(b))
