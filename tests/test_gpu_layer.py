"""The device-resident encoder layer on the GPU against the oracle, bit for
bit (NaNs compared as NaN, the one thing the contract leaves to the
hardware): each fused producer (normq, siluq, dwq) and the layer norm on
rows with zeros, constants, NaNs and infinities; the attention at tile edges
and at the model's heads; and whole layers, at small shapes and at the
model's (d_model 1024, 8 heads, ff 4096, 9 taps), in blocks of 32 and 64."""
import sys

import numpy as np
import pytest

import oracle_lib as ol
from layer_ref import attention, layer_weights, positions, unpack_packed
from libpktito_amd import synth

pytestmark = pytest.mark.gpu


def bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return np.where(np.isnan(a), np.float32(np.nan), a).view(np.uint32)


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch
    assert torch.cuda.is_available()
    return torch


def rows_with_edges(g, T, n, scale=2.0):
    """N(0, scale) + 0.5 with, when there are enough rows, a row of zeros, a
    NaN, an infinity, a constant row and a row of subnormals."""
    x = (g.standard_normal((T, n)) * scale + 0.5).astype(np.float32)
    if T >= 6:
        x[1] = 0.0
        x[2, n // 3] = np.nan
        x[3, 1] = np.inf
        x[4] = 7.0
        x[5] = np.float32(1e-40) * np.sign(x[5])
    return x


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda"))


def packed_buffers(hip, torch, n, T, qb):
    qp = torch.full((hip.packed_bytes(n, T),), -5, dtype=torch.int8, device="cuda")
    d = torch.full((T * (n // qb),), 7.0, dtype=torch.float32, device="cuda")
    return qp, d


def check_packed(qp, d, q, dd, n, T):
    assert np.array_equal(unpack_packed(qp.cpu().numpy(), n, T), q.reshape(T, n))
    assert np.array_equal(bits(d.cpu().numpy()), bits(dd))


@pytest.mark.parametrize("T,n,qb", [(1, 64, 64), (5, 1024, 32), (97, 1024, 64), (750, 1024, 32), (33, 4096, 4096),
                                    (17, 256, 256), (40, 1024, 1024), (23, 4096, 64)])
def test_normq(hip, torch, T, n, qb):
    g = synth.rng(T + n + qb)
    x = rows_with_edges(g, T, n)
    w = (1 + 0.3 * g.standard_normal(n)).astype(np.float32)
    b = (0.2 * g.standard_normal(n)).astype(np.float32)
    q, d = ol.quantize(ol.layernorm(x, w, b, 1e-5).reshape(-1), T, n, qb, n)
    qp, dt = packed_buffers(hip, torch, n, T, qb)
    say("normq", T, n, qb)
    hip.normq_dev(qp, dt, dev(torch, x), n, qb, T, dev(torch, w), dev(torch, b), 1e-5)
    torch.cuda.synchronize()
    check_packed(qp, dt, q, d, n, T)


@pytest.mark.parametrize("T,n", [(1, 64), (7, 1024), (750, 1024), (19, 4096)])
def test_layernorm(hip, torch, T, n):
    g = synth.rng(T * n)
    x = rows_with_edges(g, T, n, 3.0)
    w = (1 + 0.3 * g.standard_normal(n)).astype(np.float32)
    b = (0.2 * g.standard_normal(n)).astype(np.float32)
    want = ol.layernorm(x, w, b, 1e-5)
    xt = dev(torch, x)
    say("layernorm", T, n)
    hip.layernorm_dev(xt, T, n, dev(torch, w), dev(torch, b), 1e-5)
    torch.cuda.synchronize()
    assert np.array_equal(bits(xt.cpu().numpy()), bits(want))


@pytest.mark.parametrize("T,n,qb", [(1, 32, 32), (9, 4096, 32), (750, 4096, 64), (100, 4096, 4096), (2049, 4096, 32)])
def test_siluq(hip, torch, T, n, qb):
    """SiLU then the quantize, both kernels of the packed quantize (the
    largest case takes the one-workgroup-a-group kernel)."""
    g = synth.rng(T + 3 * n + qb)
    x = rows_with_edges(g, T, n, 4.0)
    if T >= 8:
        x[6, :] = np.float32(-90.0)            # past the exp clamp: SiLU of -90 is -0 * ...
        x[7, ::2] = np.float32(88.5)
    q, d = ol.quantize(ol.silu(x).reshape(-1), T, n, qb, n)
    qp, dt = packed_buffers(hip, torch, n, T, qb)
    say("siluq", T, n, qb)
    hip.siluq_dev(qp, dt, dev(torch, x), n, qb, T, n)
    torch.cuda.synchronize()
    say("kernel", hip.last_kernel())
    check_packed(qp, dt, q, d, n, T)


@pytest.mark.parametrize("T,D,K,qb", [(1, 64, 9, 32), (2, 128, 9, 64), (9, 128, 9, 32), (17, 1024, 9, 32),
                                      (100, 256, 31, 64), (750, 1024, 9, 64), (40, 128, 4, 32), (5, 64, 1, 64),
                                      (50, 128, 33, 32)])
def test_dwq(hip, torch, T, D, K, qb):
    """GLU, the depthwise convolution with its bias and SiLU, and the blocks'
    quantize, against the oracle's glu, dwconv and quantize."""
    g = synth.rng(T + D + K + qb)
    u = (g.standard_normal((T, 2 * D)) * 2).astype(np.float32)
    if T >= 3:
        u[1, 3] = np.inf
        u[2, D + 5] = -np.inf
    w = (0.4 * g.standard_normal((D, K))).astype(np.float32)
    b = (0.1 * g.standard_normal(D)).astype(np.float32)
    h = ol.dwconv(ol.glu(u), w, b)
    q, d = ol.quantize(h.reshape(-1), T, D, qb, D)
    qp, dt = packed_buffers(hip, torch, D, T, qb)
    say("dwq", T, D, K, qb)
    hip.dwq_dev(qp, dt, dev(torch, u), D, qb, T, dev(torch, w), dev(torch, b), K)
    torch.cuda.synchronize()
    check_packed(qp, dt, q, d, D, T)


@pytest.mark.parametrize("valu", [0, 1])
@pytest.mark.parametrize("T,D,H", [(1, 128, 2), (2, 128, 2), (7, 64, 1), (17, 128, 2), (64, 128, 2), (65, 256, 2),
                                   (130, 128, 2), (100, 1024, 8), (289, 128, 1),
                                   (37, 64, 4), (50, 128, 4), (9, 96, 2), (300, 64, 4)])
def test_attention(hip, torch, T, D, H, valu):
    """The attention's scores (with the positions' diagonals), softmax and
    weighted values against pk_k_gemm_f32 and pk_k_softmax composed on the
    CPU with the reference's panel layouts; on the matrix cores (one-step
    MFMAs) and as VALU chains. T covers one key, partial tiles and bands,
    and key counts that are not multiples of 8; heads of 16, 32 and 48
    dimensions run on the one-thread-an-output kernels."""
    g = synth.rng(T * 7 + D)
    q, k, v = (g.standard_normal((3, T, D)) * 1.5).astype(np.float32)
    p = g.standard_normal((2 * T - 1, D)).astype(np.float32)
    bu, bv = (0.3 * g.standard_normal((2, D))).astype(np.float32)
    want = attention(q, k, v, p, bu, bv, H)
    o = torch.full((T, D), 9.0, dtype=torch.float32, device="cuda")
    ws = torch.empty((hip.attention_workspace(T, H),), dtype=torch.uint8, device="cuda")
    say("attention", T, D, H, valu)
    was = hip.force_attention(valu)
    try:
        hip.attention_dev(o, dev(torch, q), dev(torch, k), dev(torch, v), dev(torch, p), dev(torch, bu),
                          dev(torch, bv), T, D, H, ws)
        torch.cuda.synchronize()
    finally:
        hip.force_attention(was)
    assert np.array_equal(bits(o.cpu().numpy()), bits(want))


@pytest.mark.parametrize("T", [37, 301])
@pytest.mark.parametrize("valu", [0, 1])
def test_attention_special_values(hip, torch, valu, T):
    """Subnormal and signed-zero operands, products past the float range and
    NaNs in the queries, keys, values and positions: every chain step's one
    rounding (an MFMA step or a v_fma_f32) gives the oracle's bits, NaNs
    compared as NaN. T = 301 takes the softmax kernel of rows over 256 keys."""
    D, H = 128, 2
    g = synth.rng(4242)
    q, k, v = (g.standard_normal((3, T, D)) * 1.5).astype(np.float32)
    p = g.standard_normal((2 * T - 1, D)).astype(np.float32)
    bu, bv = (0.3 * g.standard_normal((2, D))).astype(np.float32)
    tiny = np.float32(1e-41)
    q[3, :] = tiny * np.sign(q[3, :])          # subnormal queries: their products underflow
    k[5, ::3] = -0.0
    k[6, :] = tiny
    v[7, :] = np.float32(-1e-40)
    v[8, 10] = np.inf                          # P * inf through PV's chain
    v[13, 20] = np.nan
    q[9, 0] = np.float32(3e30)                 # a score past the float range
    k[9, 0] = np.float32(3e30)
    p[20, 4] = np.float32(2e38)
    q[11, 4] = np.float32(1e10)
    k[12, 7] = np.nan                          # a NaN score: the softmax's exp clamps it
    bu[1] = -0.0
    bv[2] = tiny
    want = attention(q, k, v, p, bu, bv, H)
    o = torch.full((T, D), 9.0, dtype=torch.float32, device="cuda")
    ws = torch.empty((hip.attention_workspace(T, H),), dtype=torch.uint8, device="cuda")
    say("attention special values", valu, T)
    was = hip.force_attention(valu)
    try:
        hip.attention_dev(o, dev(torch, q), dev(torch, k), dev(torch, v), dev(torch, p), dev(torch, bu),
                          dev(torch, bv), T, D, H, ws)
        torch.cuda.synchronize()
    finally:
        hip.force_attention(was)
    assert np.isnan(want).any() and np.isinf(want).any() and np.isfinite(want).any()
    assert np.array_equal(bits(o.cpu().numpy()), bits(want))


def run_layer(hip, torch, D, H, F, K, T, qb, seed, threads=16, tweak=None):
    g = synth.rng(seed)
    w = layer_weights(g, D=D, H=H, F=F, K=K)
    if tweak:
        tweak(w)
    x = g.standard_normal((T, D)).astype(np.float32)
    ape, ape_q, ape_d = positions(g, T, D, qb)
    R = 2 * T - 1
    lay = hip.DeviceLayer(w, torch)
    try:
        ape_qp = torch.zeros((hip.packed_bytes(D, R),), dtype=torch.int8, device="cuda")
        ape_dt = torch.empty((R * (D // qb),), dtype=torch.float32, device="cuda")
        hip.quantize_packed_dev(None, ape_qp, ape_dt, dev(torch, ape), D, R, D, qb=qb)
        ws = torch.empty((lay.workspace(T, qb),), dtype=torch.uint8, device="cuda")
        xt = dev(torch, x)
        say("layer", D, H, F, K, T, qb)
        lay.run(xt, T, ape_qp, ape_dt, qb, ws)
        torch.cuda.synchronize()
        got = xt.cpu().numpy()
        assert np.array_equal(unpack_packed(ape_qp.cpu().numpy(), D, R), ape_q.reshape(R, D))
    finally:
        lay.release()
    want = ol.conformer_layer(w, x, T, ape_q, ape_d, qb, threads=threads)
    assert np.all(np.isfinite(want))
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("T,qb", [(1, 32), (37, 64), (88, 32)])
def test_layer_small_heads(hip, torch, T, qb):
    """d_model 64 in 4 heads of 16, ff 128, 9 taps (the reference's tiny
    model's shapes): the attention on its one-thread-an-output kernels, its
    output quantized by a pass of its own; the whole layer against the
    oracle's."""
    run_layer(hip, torch, D=64, H=4, F=128, K=9, T=T, qb=qb, seed=900 + T)


@pytest.mark.parametrize("valu", [0, 1])
@pytest.mark.parametrize("T,qb", [(1, 32), (2, 64), (37, 32), (100, 64)])
def test_layer_small(hip, torch, T, qb, valu):
    """valu 0: the attention's output quantized in the PV's epilogue; valu 1:
    the VALU attention, its output written and quantized by a pass of its
    own."""
    was = hip.force_attention(valu)
    try:
        run_layer(hip, torch, 128, 2, 256, 9, T, qb, seed=T * 3 + qb)
    finally:
        hip.force_attention(was)


@pytest.mark.parametrize("T,qb", [(64, 32), (150, 64)])
def test_layer_model_shapes(hip, torch, T, qb):
    run_layer(hip, torch, 1024, 8, 4096, 9, T, qb, seed=T + qb)


@pytest.mark.parametrize("T,qb", [(750, 32), (750, 64)])
def test_layer_model_shapes_at_a_minute(hip, torch, T, qb):
    """The whole layer at the bench's size: a minute of audio (750 frames),
    d_model 1024, 8 heads, ff 4096, 9 taps, blocks of 32 (the encoder's
    default) and of 64 (its fast mode): the band of position rows and the
    750-key softmax and PV the bench times."""
    run_layer(hip, torch, 1024, 8, 4096, 9, T, qb, seed=T + qb)


@pytest.mark.parametrize("valu", [0, 1])
@pytest.mark.parametrize("qb", [32, 64])
def test_layer_attention_output_special_values(hip, torch, valu, qb):
    """Special values reaching the attention's output, which the output
    projection's activations quantize (on the matrix cores in PV's epilogue,
    valu 0; by a pass of its own after the VALU attention, valu 1): v's row
    scales planted so that head 0's channel 5 is NaN for every frame, head
    1's channel 70 infinite, head 2's channels 128..159 zero and head 3's
    192..223 subnormal, their attention outputs under 2^-121. Each block
    holding them must quantize as zeros with d = 0 (backend/ref/kernels.c:
    24-58), and the layer's output is the oracle's bit for bit."""
    def plant(w):
        s = w["v_s"]
        s[5] = np.float32(np.nan)
        s[70] = np.float32(np.inf)
        s[128:160] = 0.0
        s[192:224] = np.float32(1e-44)
    was = hip.force_attention(valu)
    try:
        run_layer(hip, torch, 256, 4, 512, 9, 37, qb, seed=91 + qb, tweak=plant)
    finally:
        hip.force_attention(was)


@pytest.mark.parametrize("qb", [32, 64])
def test_layer_narrow_heads_special_values(hip, torch, qb):
    """The same planted special values through heads 16 wide (d_model 64, 4
    heads), which take the attention's one-thread-an-output kernels: head 0's
    channel 5 NaN, head 1's channel 20 infinite, head 2 zero and head 3
    subnormal; bit for bit against the oracle."""
    def plant(w):
        s = w["v_s"]
        s[5] = np.float32(np.nan)
        s[20] = np.float32(np.inf)
        s[32:48] = 0.0
        s[48:64] = np.float32(1e-44)
    run_layer(hip, torch, 64, 4, 128, 9, 37, qb, seed=17 + qb, tweak=plant)
