"""The 24-layer chained encoder sweep (bench.py encoder_sweep, the workload
whose time is the encoder-GEMM milliseconds per audio-minute): 24 layers'
eleven products with independent weights, each product's input the
previous one's fp32 output quantized per row, run on the GPU once, and the
same chain on the oracle for sampled frames.

Every step of the chain works frame by frame (a per-row quantize, then
products whose output row t reads input row t only), so the oracle can run
the sampled frames' chain alone: from each frame's input through every
layer, in bench's order (ff1_up, ff1_down, q with k and v on its
activation, o on v's output, pw1, pw2 on the first 1024 of pw1's 2048
columns, ff2_up, ff2_down), each quantize on the row at the producer's
pitch (pw1's 2048 floats: the strided read, xs > n) and each product with
the oracle's gemm_q8 (backend/ref/kernels.c:24-86), the down projections,
o and pw2 adding to their zero-filled outputs as the GPU's do. The final
ff2_down, a mid-chain pw2 and a k output (the batched launch of q, k, v
and the positions) are compared bit for bit, and the positions'
projection on sampled rows of the encodings."""
import sys

import numpy as np
import pytest

import oracle_lib as ol
from libpktito_amd import synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch
    assert torch.cuda.is_available()
    return torch


def product(p, x):
    """The oracle's p of the rows x [F, xs] (the first p.K floats of each
    row quantized per row), added to zeros where p adds."""
    F, xs = x.shape
    q, d = ol.quantize(np.ascontiguousarray(x).reshape(-1), F, p.K, p.K, xs)
    out = np.zeros(F * p.N, np.float32)
    ol.gemm_q8(out, p.N, p.w, p.ws, None, p.N, q, d, p.K, p.K, F, p.add, threads=16)
    return out.reshape(F, p.N)


@pytest.mark.parametrize("M", [750, 7500])
def test_encoder_chain_against_the_oracle(hip, torch, M):
    import bench
    say("chain build", M)
    fn, ops, layers = bench.encoder_sweep(hip, torch, M, seed=10 + M)
    say("chain run", M)
    fn()
    torch.cuda.synchronize()
    F = np.unique(np.concatenate([[0, M - 1], synth.rng(M + 5).integers(0, M, 6)]))
    x = layers[0]["ff1_up"].x.cpu().numpy()[F]
    mid = len(layers) // 2
    for L, lay in enumerate(layers):
        say("oracle layer", L)
        h = product(lay["ff1_up"], x)
        fd = product(lay["ff1_down"], h)
        k = product(lay["k"], fd)
        v = product(lay["v"], fd)
        o = product(lay["o"], v)
        p1 = product(lay["pw1"], o)
        p2 = product(lay["pw2"], p1)            # the first 1024 of 2048 floats a row: xs > n
        u = product(lay["ff2_up"], p2)
        x = product(lay["ff2_down"], u)
        if L == mid:
            got = lay["pw2"].out.cpu().numpy()[F]
            assert np.array_equal(bits(got), bits(p2)), f"pw2 of layer {L}"
            got = lay["k"].out.cpu().numpy()[F]
            assert np.array_equal(bits(got), bits(k)), f"k of layer {L}"
    got = layers[-1]["ff2_down"].out.cpu().numpy()[F]
    # live values: finite (they grow about 1.17 times a layer, which the
    # per-row quantize does not see) and almost none zero
    assert np.isfinite(got).all() and np.count_nonzero(got) > 0.99 * got.size
    assert np.array_equal(bits(got), bits(x)), "the last layer's ff2_down"
    # the positions' projection (its own input, the encodings, quantized once)
    pos = layers[-1]["pos"]
    R = 2 * M - 1
    rows = np.unique(np.concatenate([[0, R - 1], synth.rng(R).integers(0, R, 6)]))
    enc = pos.x.cpu().numpy()[rows]
    got = pos.out.cpu().numpy()[rows]
    assert np.array_equal(bits(got), bits(product(pos, enc))), "pos"
    for lay in layers:
        for p in lay.values():
            p.m.release()
