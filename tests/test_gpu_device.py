"""The device-resident path (activations and outputs in HBM, asynchronous on a
stream) and the grouped launch, against the oracle bit for bit: the shapes
of one FastConformer layer at a minute of audio and at ten minutes, and a
ragged batch of segments in one launch."""
import sys
import zlib

import numpy as np
import pytest

import oracle_lib as ol
from layer_ref import unpack_packed
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


def sampled_oracle(q, d, w, ws, bias, K, N, frames, add=0, old=None):
    """The oracle's outputs for the given frames only (a sub-act of them)."""
    idx = np.asarray(frames)
    qs = np.ascontiguousarray(q.reshape(-1, K)[idx]).reshape(-1)
    ds = np.ascontiguousarray(d[idx])
    out = old[idx].reshape(-1).copy() if old is not None else np.zeros(len(idx) * N, np.float32)
    ol.gemm_q8(out, N, w, ws, bias, N, qs, ds, K, K, len(idx), add, threads=16)
    return out.reshape(len(idx), N)


def run_product(pk, torch, name, M, K, N, half, add, seed, sample=64):
    g = synth.rng(seed)
    wr = synth.weights(g, N, K)
    w = synth.pack_q8(wr)
    ws = synth.scales(g, N)
    x = synth.activations(g, M, K, half)
    old = g.standard_normal((M, N)).astype(np.float32) if add else None
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    qt = torch.empty((M, K), dtype=torch.int8, device=dev)
    dt = torch.empty((M,), dtype=torch.float32, device=dev)
    ot = torch.from_numpy(old).to(dev) if add else torch.empty((M, N), dtype=torch.float32, device=dev)
    say("device product", name, M, K, N, add)
    with pk.Q8Matrix(w, ws) as m:
        pk.quantize_dev(qt, dt, xt, K, K, M, K)
        pk.gemm_q8_dev(ot, N, m, 0, N, None, None, qt, dt, K, K, M, add, ws_ptr=m.dev_scales)
        torch.cuda.synchronize()
        say("kernel", pk.last_kernel())
    q = qt.cpu().numpy().reshape(-1)
    d = dt.cpu().numpy()
    out = ot.cpu().numpy()
    q2, d2 = ol.quantize(x.reshape(-1), M, K, K, K)
    assert np.array_equal(q, q2) and np.array_equal(bits(d), bits(d2)), name
    frames = np.unique(np.concatenate([[0, M - 1], synth.rng(seed + 1).integers(0, M, sample)]))
    want = sampled_oracle(q, d, w, ws, None, K, N, frames, add, old)
    assert np.array_equal(bits(out[frames]), bits(want)), name


@pytest.mark.parametrize("prod", synth.layer_products(750), ids=lambda p: p[0])
def test_layer_products_minute(hip, torch, prod):
    name, M, K, N, half, add = prod
    run_product(hip, torch, name, M, K, N, half, int(add), seed=zlib.crc32(name.encode()) % 1000)


@pytest.mark.parametrize("prod", [p for p in synth.layer_products(7500) if p[0] in ("ff1_up", "ff1_down", "pos", "pw1")],
                         ids=lambda p: p[0])
def test_layer_products_ten_minutes(hip, torch, prod):
    name, M, K, N, half, add = prod
    run_product(hip, torch, name, M, K, N, half, int(add), seed=17 + len(name), sample=48)


@pytest.mark.parametrize("K,N", [(1024, 4096), (4096, 1024)])
def test_ragged_batch_grouped(hip, torch, K, N):
    """Eight segments of 150-750 frames (12-60 s) in one launch: each
    segment's outputs are the bits of its own product, and the oracle's; and
    the same grouped launch under every tiling forced (the 128 x 128 and
    larger tiles store whole lines from consecutive lanes across segment
    ends)."""
    lens = synth.ragged_lengths()
    g = synth.rng(K + N)
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    dev = torch.device("cuda")
    segs, solo, host = [], [], []
    with hip.Q8Matrix(w, ws) as m:
        for L in lens:
            x = synth.activations(g, L, K)
            q, d = ol.quantize(x.reshape(-1), L, K, K, K)
            qt = torch.from_numpy(q.reshape(L, K)).to(dev)
            dt = torch.from_numpy(d).to(dev)
            ot = torch.full((L, N), 7.0, dtype=torch.float32, device=dev)
            o2 = torch.full((L, N), 7.0, dtype=torch.float32, device=dev)
            segs.append((ot, N, qt, dt, K, K, L))
            solo.append((o2, qt, dt, L))
            host.append((q, d, L))
        say("grouped", lens, K, N)
        hip.gemm_q8_grouped_dev(m, 0, N, m.dev_scales, None, segs, 0)
        for o2, qt, dt, L in solo:
            hip.gemm_q8_dev(o2, N, m, 0, N, None, None, qt, dt, K, K, L, 0, ws_ptr=m.dev_scales)
        torch.cuda.synchronize()
        for (ot, _, _, _, _, _, L), (o2, _, _, _), (q, d, _) in zip(segs, solo, host):
            a, b = ot.cpu().numpy(), o2.cpu().numpy()
            assert np.array_equal(bits(a), bits(b))
            frames = np.unique(np.concatenate([[0, L - 1], synth.rng(L).integers(0, L, 24)]))
            want = sampled_oracle(q, d, w, ws, None, K, N, frames)
            assert np.array_equal(bits(a[frames]), bits(want))
        # the grouped launch under every tiling forced (each segment's own
        # launch above, checked against the oracle, is the reference)
        try:
            for ti in range(hip.tilings()):
                hip.force_tiling(ti)
                for (ot, *_rest) in segs:
                    ot.fill_(7.0)
                say("grouped forced", ti, K, N)
                hip.gemm_q8_grouped_dev(m, 0, N, m.dev_scales, None, segs, 0)
                torch.cuda.synchronize()
                for j, ((ot, *_r1), (o2, *_r2)) in enumerate(zip(segs, solo)):
                    assert torch.equal(ot.view(torch.int32), o2.view(torch.int32)), (ti, j, hip.last_kernel())
        finally:
            hip.force_tiling(-1)


def test_interior_panels_device(hip, torch):
    """A run of panels from the middle of an uploaded matrix (r0 > 0) on the
    device path, with bias and add, at an odd output stride."""
    g = synth.rng(99)
    M, K, N = 200, 1024, 512
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    bias = g.standard_normal(N).astype(np.float32)
    x = synth.activations(g, M, K).reshape(-1)
    q, d = ol.quantize(x, M, K, K, K)
    os_ = N + 5
    old = g.standard_normal(M * os_).astype(np.float32)
    r0, rows = 144, 240
    want = old.copy()
    ol.gemm_q8(want, os_, w, ws, bias, rows, q, d, K, K, M, 1, r0=r0)
    dev = torch.device("cuda")
    ot = torch.from_numpy(old).to(dev)
    qt, dt = torch.from_numpy(q).to(dev), torch.from_numpy(d).to(dev)
    bt = torch.from_numpy(bias).to(dev)
    wst = torch.from_numpy(ws).to(dev)
    say("interior panels", r0, rows)
    with hip.Q8Matrix(w, ws) as m:
        hip.gemm_q8_dev(None, os_, m, r0, rows, None, None, qt, dt, K, K, M, 1,
                        ws_ptr=wst.data_ptr() + 4 * r0, out_ptr=ot.data_ptr() + 4 * r0)
        torch.cuda.synchronize()
        # the same with a bias (its pointer at row r0)
        ot2 = torch.from_numpy(old).to(dev)
        import libpktito_amd as pk
        a = pk.Act(qt.data_ptr(), dt.data_ptr(), K, K, M)
        import ctypes
        rc = pk.lib().pk_hip_gemm_q8_dev(ot2.data_ptr() + 4 * r0, os_, m.handle, r0, rows,
                                         wst.data_ptr() + 4 * r0, bt.data_ptr() + 4 * r0,
                                         ctypes.byref(a), 1, 0, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
    assert np.array_equal(bits(ot2.cpu().numpy()), bits(want))
    want_nob = old.copy()
    ol.gemm_q8(want_nob, os_, w, ws, None, rows, q, d, K, K, M, 1, r0=r0)
    assert np.array_equal(bits(ot.cpu().numpy()), bits(want_nob))


@pytest.mark.parametrize("M,K,N", [(750, 1024, 4096), (1499, 1024, 1024), (300, 4096, 1024), (16, 1024, 4096),
                                   (5, 640, 1040), (97, 640, 208)])
def test_packed_path(hip, torch, M, K, N):
    """The packed-activation path: its q and d are the oracle's, its packed
    copy holds the same bytes, and every tiling's products are the bits of
    the row-major path and of the oracle."""
    g = synth.rng(M * 3 + K)
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    x = synth.activations(g, M, K)
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    qt = torch.empty((M, K), dtype=torch.int8, device=dev)
    dt = torch.empty((M,), dtype=torch.float32, device=dev)
    qp = torch.zeros((hip.packed_bytes(K, M),), dtype=torch.int8, device=dev)
    say("packed quantize", M, K, N)
    hip.quantize_packed_dev(qt, qp, dt, xt, K, M, K)
    torch.cuda.synchronize()
    q, d = ol.quantize(x.reshape(-1), M, K, K, K)
    assert np.array_equal(qt.cpu().numpy().reshape(-1), q) and np.array_equal(bits(dt.cpu().numpy()), bits(d))
    assert np.array_equal(unpack_packed(qp.cpu().numpy(), K, M), q.reshape(M, K))
    frames = np.unique(np.concatenate([[0, M - 1], synth.rng(M).integers(0, M, 32)]))
    want = sampled_oracle(q, d, w, ws, None, K, N, frames)
    with hip.Q8Matrix(w, ws) as m:
        ref = torch.empty((M, N), dtype=torch.float32, device=dev)
        hip.gemm_q8_dev(ref, N, m, 0, N, None, None, qt, dt, K, K, M, 0, ws_ptr=m.dev_scales)
        torch.cuda.synchronize()
        r = ref.cpu().numpy()
        assert np.array_equal(bits(r[frames]), bits(want))
        try:
            for ti in [-1] + list(range(hip.tilings())):
                hip.force_tiling(ti)
                out = torch.full((M, N), 3.0, dtype=torch.float32, device=dev)
                say("packed product", ti, M, K, N)
                hip.gemm_q8_packed_dev(out, N, m, 0, N, m.dev_scales, None, qp, dt, K, M, 0)
                torch.cuda.synchronize()
                assert np.array_equal(bits(out.cpu().numpy()), bits(r)), (ti, hip.last_kernel())
        finally:
            hip.force_tiling(-1)


@pytest.mark.parametrize("qb", [None, 32, 64])
@pytest.mark.parametrize("K", [1024, 4096, 128])
def test_batch_of_products(hip, torch, K, qb):
    """Independent products in one launch (the attention's q, k, v and the
    positions' projection at once): each job's outputs are the bits its own
    launch gives, with jobs of different frame counts, channel counts, a run
    of interior panels, bias and add, per-row or in blocks of 32 or 64; under
    the heuristic and under every tiling (short inputs, and tilings without
    a blocked batch, fall back to one launch a job)."""
    nb = 1 if qb is None else K // qb
    dev = torch.device("cuda")
    g = synth.rng(K + 17)
    specs = [(37, 1024, 0, 1024, False, 0), (750, 1024, 0, 1024, True, 1), (1, 512, 0, 512, False, 0),
             (1499, 1040, 16, 1008, True, 0), (0, 256, 0, 256, False, 0), (200, 2048, 32, 96, False, 1)]
    mats, jobs, singles = [], [], []
    for (T, N, r0, rows, use_bias, add) in specs:
        w = synth.pack_q8(synth.weights(g, N, K))
        ws = synth.scales(g, N)
        m = hip.Q8Matrix(w, ws)
        mats.append(m)
        x = torch.from_numpy(synth.activations(g, max(T, 1), K)).to(dev)
        qp = torch.zeros((hip.packed_bytes(K, max(T, 1)),), dtype=torch.int8, device=dev)
        d = torch.empty((max(T, 1) * nb,), dtype=torch.float32, device=dev)
        if T:
            hip.quantize_packed_dev(None, qp, d, x, K, T, K, qb=K if qb is None else qb)
        bias = torch.from_numpy(g.standard_normal(N).astype(np.float32)).to(dev) if use_bias else None
        os_ = N + 3
        base = torch.from_numpy(g.standard_normal(max(T, 1) * os_).astype(np.float32)).to(dev)
        ws_ptr = m.dev_scales + 4 * r0
        bias_v = bias[r0:] if bias is not None else None
        singles.append((base, os_, m, r0, rows, ws_ptr, bias_v, qp, d, T, add))
    torch.cuda.synchronize()
    want = []
    for (base, os_, m, r0, rows, ws_ptr, bias_v, qp, d, T, add) in singles:
        out = base.clone()
        if T:
            hip.gemm_q8_packed_dev(None, os_, m, r0, rows, ws_ptr, bias_v, qp, d, K, T, add,
                                   out_ptr=out.data_ptr() + 4 * r0, qb=K if qb is None else qb)
        want.append(out)
    torch.cuda.synchronize()
    try:
        for ti in [-1] + list(range(hip.tilings())):
            hip.force_tiling(ti)
            outs = [b.clone() for (b, *_rest) in singles]
            jobs = []
            for o, (base, os_, m, r0, rows, ws_ptr, bias_v, qp, d, T, add) in zip(outs, singles):
                jobs.append((o[r0:], os_, m, r0, rows, ws_ptr, bias_v, qp, d, K, T, add))
            say("batch", K, qb, ti)
            hip.gemm_q8_batch_dev(jobs, qb=qb)
            torch.cuda.synchronize()
            for j, (o, wnt) in enumerate(zip(outs, want)):
                assert np.array_equal(bits(o.cpu().numpy()), bits(wnt.cpu().numpy())), (ti, j, hip.last_kernel())
    finally:
        hip.force_tiling(-1)
        for m in mats:
            m.release()


BLOCKED = [(qb, M, K, N) for (M, K, N) in [(750, 1024, 1024), (300, 4096, 1024), (37, 1056, 208), (129, 512, 64),
                                           (1499, 1024, 96)]
           for qb in (32, 64) if K % qb == 0]


@pytest.mark.parametrize("qb,M,K,N", BLOCKED)
def test_blocked_products(hip, torch, qb, M, K, N):
    """The encoder's blocks (qb 32 and 64) on the pipelined tiles: the packed
    quantize's q, d and packed bytes are the oracle's, and the product of every
    tiling with a blocked variant, packed and row-major, with bias and add,
    under each rounding mode, is the oracle's, bit for bit. K = 1056 has an
    odd number of 32-input blocks and a padding unit past them."""
    import ctypes.util
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    g = synth.rng(M + K + N + qb)
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    bias = g.standard_normal(N).astype(np.float32)
    x = synth.activations(g, M, K)
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    qt = torch.empty((M, K), dtype=torch.int8, device=dev)
    dt = torch.empty((M * K // qb,), dtype=torch.float32, device=dev)
    qp = torch.zeros((hip.packed_bytes(K, M),), dtype=torch.int8, device=dev)
    say("blocked quantize", qb, M, K, N)
    hip.quantize_packed_dev(qt, qp, dt, xt, K, M, K, qb=qb)
    torch.cuda.synchronize()
    q, d = ol.quantize(x.reshape(-1), M, K, qb, K)
    assert np.array_equal(qt.cpu().numpy().reshape(-1), q) and np.array_equal(bits(dt.cpu().numpy()), bits(d))
    assert np.array_equal(unpack_packed(qp.cpu().numpy(), K, M), q.reshape(M, K))
    base = g.standard_normal(M * N).astype(np.float32)
    bt = torch.from_numpy(bias).to(dev)
    modes = {0: 0, 1: 0x800, 2: 0x400, 3: 0xC00}
    with hip.Q8Matrix(w, ws) as m:
        try:
            for rm in (0, 1, 2):
                want = base.copy()
                assert libm.fesetround(modes[rm]) == 0
                try:
                    ol.gemm_q8(want, N, w, ws, bias, N, q, d, K, qb, M, 1, threads=16)
                finally:
                    libm.fesetround(0)
                for ti in [-1, 4, 5, 6]:
                    hip.force_tiling(ti)
                    for packed in (True, False):
                        out = torch.from_numpy(base).to(dev)
                        say("blocked product", qb, M, K, N, rm, ti, packed)
                        if packed:
                            hip.gemm_q8_packed_dev(out, N, m, 0, N, m.dev_scales, bt, qp, dt, K, M, 1, rmode=rm,
                                                   qb=qb)
                        else:
                            hip.gemm_q8_dev(out, N, m, 0, N, None, bt, qt, dt, K, qb, M, 1, rmode=rm,
                                            ws_ptr=m.dev_scales)
                        torch.cuda.synchronize()
                        assert hip.last_kernel().startswith("pipe"), hip.last_kernel()
                        assert np.array_equal(bits(out.cpu().numpy().reshape(-1)), bits(want)), \
                            (qb, M, K, N, rm, ti, packed, hip.last_kernel())
        finally:
            hip.force_tiling(-1)


def special_rows(x):
    """Columns the block rule zeroes or scales at its edges: all zeros, a NaN,
    an infinity, every magnitude below 2^-121 (zeroed), and a largest
    magnitude of exactly 2^-121 (kept, with a subnormal scale)."""
    T, n = x.shape
    if T >= 6:
        x[1] = 0.0
        x[2, n // 2] = np.nan
        x[3, n - 1] = -np.inf
        x[4] = np.sign(x[4]) * np.float32(2.0 ** -122)
        x[5] = x[5] * np.float32(2.0 ** -125)
        x[5, 7] = np.float32(2.0 ** -121)
    return x


@pytest.mark.parametrize("T,n,qb", [(1, 32, 32), (5, 640, 640), (97, 608, 608), (97, 1056, 32), (17, 4096, 64),
                                    (300, 4096, 4096), (300, 4096, 64), (750, 1024, 32), (2000, 4096, 4096),
                                    (1800, 4096, 32), (7500, 1024, 1024), (2249, 4096, 64)])
def test_packed_quantize_kernels(hip, torch, T, n, qb):
    """The packed quantize kernels (one wave a column, or a wave a
    1024-input chunk of a wide column in blocks; one workgroup a half
    16-column group) and the
    choice by size: q, d and the packed bytes are
    the oracle's, with and without the row-major copy, over a packed buffer
    that held other bytes before."""
    g = synth.rng(T * 7 + n + qb)
    x = special_rows(synth.activations(g, T, n))
    q, d = ol.quantize(x.reshape(-1), T, n, qb, n)
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    big = T * n >= (9 << 20 if n > 1024 else 5 << 20)
    try:
        for kind in (-1, 0, 1, 2):
            hip.force_quantize(kind)
            for with_q in (True, False):
                qt = torch.full((T, n), 77, dtype=torch.int8, device=dev) if with_q else None
                dt = torch.full((T * n // qb,), 5.0, dtype=torch.float32, device=dev)
                qp = torch.full((hip.packed_bytes(n, T),), -3, dtype=torch.int8, device=dev)
                say("packed quantize", T, n, qb, kind, with_q)
                hip.quantize_packed_dev(qt, qp, dt, xt, n, T, n, qb=qb)
                torch.cuda.synchronize()
                want = ("quant_group" if kind == 1 or (kind == -1 and big) else "quant_wave" if kind == 2 else
                        "quant_chunk" if qb != n and n > 1024 else "quant_wave")
                assert hip.last_kernel().startswith(want), (kind, hip.last_kernel())
                if with_q:
                    assert np.array_equal(qt.cpu().numpy().reshape(-1), q)
                assert np.array_equal(bits(dt.cpu().numpy()), bits(d))
                assert np.array_equal(unpack_packed(qp.cpu().numpy(), n, T), q.reshape(T, n))
    finally:
        hip.force_quantize(-1)


STRIDED = [(n, xs, qb) for (n, xs) in [(1024, 1056), (1024, 2048), (96, 128), (4096, 4128), (640, 704)]
           for qb in (None, 32, 64) if qb is None or n % qb == 0]


@pytest.mark.parametrize("n,xs,qb", STRIDED)
def test_quantize_reads_columns_at_a_stride(hip, torch, n, xs, qb):
    """quantize_dev and quantize_packed_dev with xs > n: column t's inputs at
    x + t xs (backend/kernels.h:47-58), the floats between one column's n
    and the next left unread, as kcheck draws xs = n + 32 (tests/kcheck.c:
    98-118) and the chained encoder reads the first 1024 of pw1's 2048
    outputs a row. The floats past n hold NaN and huge values, so a kernel
    that read them would zero the block or change its scale."""
    qbv = n if qb is None else qb
    g = synth.rng(n * 7 + xs + qbv)
    dev = torch.device("cuda")
    for T in (1, 37, 750):
        x = synth.activations(g, T, xs)
        x[:, n:] = np.float32(np.nan)
        x[::3, n:] = np.float32(3e38)
        q, d = ol.quantize(x.reshape(-1), T, n, qbv, xs)
        xt = torch.from_numpy(x).to(dev)
        qt = torch.empty((T, n), dtype=torch.int8, device=dev)
        dt = torch.empty((T * (n // qbv),), dtype=torch.float32, device=dev)
        say("strided quantize", n, xs, qbv, T)
        hip.quantize_dev(qt, dt, xt, n, qbv, T, xs)
        torch.cuda.synchronize()
        assert np.array_equal(qt.cpu().numpy().reshape(-1), q), (n, xs, qbv, T)
        assert np.array_equal(bits(dt.cpu().numpy()), bits(d)), (n, xs, qbv, T)
        if qb in (None, 32, 64) and n <= 4096:
            qp = torch.zeros((hip.packed_bytes(n, T),), dtype=torch.int8, device=dev)
            qt2 = torch.empty((T, n), dtype=torch.int8, device=dev)
            dt2 = torch.empty_like(dt)
            say("strided packed quantize", n, xs, qbv, T)
            hip.quantize_packed_dev(qt2, qp, dt2, xt, n, T, xs, qb=qb)
            torch.cuda.synchronize()
            assert np.array_equal(qt2.cpu().numpy().reshape(-1), q), (n, xs, qbv, T)
            assert np.array_equal(bits(dt2.cpu().numpy()), bits(d)), (n, xs, qbv, T)
            assert np.array_equal(unpack_packed(qp.cpu().numpy(), n, T), q.reshape(T, n))


SPLIT_SHAPES = [(M, K, N) for M in (1, 4, 16) for (K, N) in ((1024, 4096), (4096, 1024), (640, 1040))] + \
    [(7, 96, 64), (16, 3136, 256)]


@pytest.mark.parametrize("M,K,N", SPLIT_SHAPES)
def test_split_few_frame_products(hip, torch, M, K, N):
    """The few-frame products split over K (pk_hip_gemm_q8_ws_dev and its
    packed form): under every forced split and the automatic one, row-major
    and packed, with bias and add, a run of interior panels, os = 0 at one
    frame, the bits of the unsplit entry, which the oracle pins here too;
    two calls in a row on one workspace (the counters the first leaves must
    be zero for the second), and the counters zero after every call."""
    g = synth.rng(M * 13 + K + N)
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    bias = g.standard_normal(N).astype(np.float32)
    x = synth.activations(g, M, K)
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    qt = torch.empty((M, K), dtype=torch.int8, device=dev)
    dt = torch.empty((M,), dtype=torch.float32, device=dev)
    qp = torch.zeros((hip.packed_bytes(K, M),), dtype=torch.int8, device=dev)
    hip.quantize_packed_dev(qt, qp, dt, xt, K, M, K)
    r0 = 16 if N > 64 else 0
    rows = N - r0
    os_ = 0 if M == 1 else N + 3
    bt = torch.from_numpy(bias).to(dev)
    base = torch.from_numpy(g.standard_normal(max(1, M * os_ + N)).astype(np.float32)).to(dev)
    q, d = ol.quantize(x.reshape(-1), M, K, K, K)
    want_host = base.cpu().numpy().copy()
    ol.gemm_q8(want_host, os_, w, ws, bias, rows, q, d, K, K, M, 1, r0=r0, threads=16)
    work = torch.zeros((hip.gemm_workspace(rows),), dtype=torch.uint8, device=dev)
    counters = (rows // 16 * 4 + 255) // 256 * 256        # a counter a panel, first in the workspace
    with hip.Q8Matrix(w, ws) as m:
        ref = base.clone()
        hip.gemm_q8_dev(None, os_, m, r0, rows, None, bt[r0:], qt, dt, K, K, M, 1,
                        ws_ptr=m.dev_scales + 4 * r0, out_ptr=ref.data_ptr() + 4 * r0)
        torch.cuda.synchronize()
        assert np.array_equal(bits(ref.cpu().numpy()), bits(want_host))
        try:
            for sp in (-1, 1, 2, 3, 4, 5, 8):
                hip.force_split(sp)
                for packed in (False, True):
                    for call in range(2):
                        out = base.clone()
                        say("split product", M, K, N, sp, packed, call)
                        if packed:
                            hip.gemm_q8_packed_dev(None, os_, m, r0, rows, m.dev_scales + 4 * r0, bt[r0:], qp, dt,
                                                   K, M, 1, out_ptr=out.data_ptr() + 4 * r0, work=work)
                        else:
                            hip.gemm_q8_dev(None, os_, m, r0, rows, None, bt[r0:], qt, dt, K, K, M, 1,
                                            ws_ptr=m.dev_scales + 4 * r0, out_ptr=out.data_ptr() + 4 * r0,
                                            work=work)
                        torch.cuda.synchronize()
                        kn = hip.last_kernel()
                        assert np.array_equal(bits(out.cpu().numpy()), bits(want_host)), (sp, packed, call, kn)
                        assert int(work[:counters].count_nonzero()) == 0, (sp, packed, call, kn)
        finally:
            hip.force_split(-1)


def test_split_workspace_refusals(hip, torch):
    """A workspace too small or misaligned is refused before anything runs."""
    g = synth.rng(3)
    w = synth.pack_q8(synth.weights(g, 1024, 256))
    ws = synth.scales(g, 1024)
    dev = torch.device("cuda")
    q = torch.zeros((1, 256), dtype=torch.int8, device=dev)
    d = torch.ones((1,), dtype=torch.float32, device=dev)
    out = torch.zeros((1024,), dtype=torch.float32, device=dev)
    need = hip.gemm_workspace(1024)
    assert need >= 1024 // 16 * 8 * 1024
    small = torch.zeros((need - 256,), dtype=torch.uint8, device=dev)
    big = torch.zeros((need + 256,), dtype=torch.uint8, device=dev)
    with hip.Q8Matrix(w, ws) as m:
        with pytest.raises(hip.PkHipError):
            hip.gemm_q8_dev(out, 0, m, 0, 1024, None, None, q, d, 256, 256, 1, 0, ws_ptr=m.dev_scales, work=small)
        with pytest.raises(hip.PkHipError):
            hip.gemm_q8_dev(None, 0, m, 0, 1024, None, None, q, d, 256, 256, 1, 0, ws_ptr=m.dev_scales,
                            out_ptr=out.data_ptr(), work=big[16:])
    torch.cuda.synchronize()


@pytest.mark.parametrize("M", [1, 16])
def test_split_deep_products_split_by_themselves(hip, torch, M):
    """Deep few-panel products (K = 8192 into 512 channels at 16 frames, K =
    16384 at one) take the split without forcing; their bits are the unsplit
    entry's and, through the host entry (the lease's own workspace), the
    oracle's."""
    K = 8192 if M == 16 else 16384
    N = 512
    g = synth.rng(M + K)
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    x = synth.activations(g, M, K)
    dev = torch.device("cuda")
    xt = torch.from_numpy(x).to(dev)
    qt = torch.empty((M, K), dtype=torch.int8, device=dev)
    dt = torch.empty((M,), dtype=torch.float32, device=dev)
    hip.quantize_dev(qt, dt, xt, K, K, M, K)
    q, d = ol.quantize(x.reshape(-1), M, K, K, K)
    want = np.zeros(M * N, np.float32)
    ol.gemm_q8(want, N, w, ws, None, N, q, d, K, K, M, 0, threads=16)
    work = torch.zeros((hip.gemm_workspace(N),), dtype=torch.uint8, device=dev)
    with hip.Q8Matrix(w, ws) as m:
        for call in range(2):
            out = torch.zeros((M, N), dtype=torch.float32, device=dev)
            say("deep split product", M, K, N, call)
            hip.gemm_q8_dev(out, N, m, 0, N, None, None, qt, dt, K, K, M, 0, ws_ptr=m.dev_scales, work=work)
            torch.cuda.synchronize()
            assert "split 4" in hip.last_kernel(), hip.last_kernel()
            assert np.array_equal(bits(out.cpu().numpy().reshape(-1)), bits(want)), call
        host = np.zeros(M * N, np.float32)
        say("deep split product, host entry", M, K, N)
        hip.gemm_q8(host, N, w, ws, None, N, hip.make_act(q, d, K, K, M), 0)
        assert "split" in hip.last_kernel(), hip.last_kernel()
        assert np.array_equal(bits(host), bits(want))


STREAM_SHAPES = [(1100, 1024, 2048, 0, 0), (4100, 640, 4096, 1, 1), (2999, 2048, 1040, 1, 4), (777, 4096, 512, 0, 1)]


@pytest.mark.parametrize("M,K,N,add,pad", STREAM_SHAPES)
def test_streamed_tiles_walk_every_tile(hip, torch, M, K, N, add, pad):
    """Every streamed tiling forced on products whose tiles do not fill the
    persistent grid evenly (fewer tiles than workgroups, several rounds with
    a remainder, a partial last channel tile, K = 640 whose units are not a
    multiple of four), with bias, with and without add, at output strides
    with and without 16-byte rows (os = N + pad), on packed and row-major
    activations: every output bit for bit the per-launch pipelined tile's
    (itself held to the oracle on these shapes' frames sampled here)."""
    g = synth.rng(M + K + N + pad)
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    bias = g.standard_normal(N).astype(np.float32)
    x = synth.activations(g, M, K).reshape(-1)
    q, d = ol.quantize(x, M, K, K, K)
    os_ = N + pad
    old = g.standard_normal(M * os_).astype(np.float32)
    dev = torch.device("cuda")
    qt = torch.from_numpy(q.reshape(M, K)).to(dev)
    dt = torch.from_numpy(d).to(dev)
    bt = torch.from_numpy(bias).to(dev)
    qp = torch.empty((hip.packed_bytes(K, M),), dtype=torch.int8, device=dev)
    names = [hip.tiling_name(i) for i in range(hip.tilings())]
    pipe = names.index("pipe<128x128w8,1,4>")
    streams = [i for i, n in enumerate(names) if n.startswith("stream")]
    assert streams
    outs = {}
    try:
        with hip.Q8Matrix(w, ws) as m:
            xt = torch.from_numpy(x.reshape(M, K)).to(dev)
            dp = torch.empty((M,), dtype=torch.float32, device=dev)
            hip.quantize_packed_dev(None, qp, dp, xt, K, M, K)
            for ti in [pipe] + streams:
                hip.force_tiling(ti)
                for packed in (False, True):
                    say("streamed walk", names[ti], M, K, N, add, pad, "packed" if packed else "rows")
                    ot = torch.from_numpy(old.reshape(M, os_)).to(dev)
                    if packed:
                        hip.gemm_q8_packed_dev(None, os_, m, 0, N, m.dev_scales, bt, qp, dp, K, M, add,
                                               out_ptr=ot.data_ptr())
                    else:
                        hip.gemm_q8_dev(ot, os_, m, 0, N, None, bt, qt, dt, K, K, M, add, ws_ptr=m.dev_scales)
                    torch.cuda.synchronize()
                    assert hip.last_kernel() == names[ti], (hip.last_kernel(), names[ti])
                    outs[(ti, packed)] = ot.cpu().numpy().reshape(M, os_)
    finally:
        hip.force_tiling(-1)
    ref = outs[(pipe, False)]
    frames = np.unique(np.concatenate([[0, M - 1], synth.rng(M).integers(0, M, 24)]))
    want = sampled_oracle(q, d, w, ws, bias, K, N, frames, add, old.reshape(M, os_)[:, :N] if add else None)
    assert np.array_equal(bits(ref[frames, :N]), bits(want))
    for key, o in outs.items():
        assert np.array_equal(bits(o), bits(ref)), (names[key[0]], key[1])
