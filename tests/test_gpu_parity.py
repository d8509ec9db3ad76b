"""The HIP path against the oracle and the reference's fixtures, bit for bit.

Every comparison is of raw bits (memcmp, as the reference's tests/kcheck.c:77-94
compares): the int8 activations, the block scales and every fp32 output,
including the floats between one column's outputs and the next. All calls
go through the C ABI (libpkhip.so) via libpktito_amd.
"""
import ctypes
import ctypes.util
import sys
import threading

import numpy as np
import pytest

import cases
import oracle_lib as ol
from libpktito_amd import synth

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def same(a, b):
    return np.array_equal(bits(np.asarray(a, np.float32)), bits(np.asarray(b, np.float32)))


def hip_quantize(pk, x, T, n, qb, xs):
    q = np.full(T * n, 99, np.int8)
    d = np.full(T * (n // qb), 99.0, np.float32)
    a = pk.make_act(q, d, n, qb, T)
    pk.quantize(a, x, xs)
    return q, d


# ------------------------------------------------- against the reference ---

def test_quantize_reference_fixtures(hip):
    man, qz, _ = cases.golden()
    for name, x, T, n, qb, xs in cases.golden_quant_cases():
        say("quantize fixture", name, T, n, qb)
        q, d = hip_quantize(hip, x, T, n, qb, xs)
        assert np.array_equal(q, qz[f"{name}_q"]), name
        assert same(d, qz[f"{name}_d"]), name


def test_gemm_reference_fixtures(hip):
    man, _, gz = cases.golden()
    acts = {m["name"]: m["act"] for m in man["gemm"]}
    for g in cases.golden_gemm_cases():
        n, T, qb = g["n"], g["T"], g["qb"]
        say("gemm fixture", g["name"], g["rows"], n, T, qb)
        if "q" not in g:
            g["q"], g["d"] = hip_quantize(hip, g["x"], T, n, qb, n)
            assert cases.digest(g["q"], g["d"]) == acts[g["name"]], g["name"]
        out = g["out0"].copy()
        with hip.Q8Matrix(g["w"], g["ws"]):
            a = hip.make_act(g["q"], g["d"], n, qb, T)
            r0 = g["r0"]
            bias = g["bias"][r0:] if g["bias"] is not None else None
            hip.gemm_q8(out, g["os"], g["w"], g["ws"][r0:], bias, g["rows"] - r0, a, g["add"],
                        w_offset=r0 * n, out_offset=r0)
        assert same(out, gz[g["name"]]), g["name"]


# ------------------------------------------------- against the oracle ---

def test_gemm_random_against_oracle(hip):
    for p in cases.gemm_random_params(160, seed=4321):
        g = cases.gemm_case(p["seed"] + 90000, p["rows"], p["n"], p["T"], p["qb"], p["add"], p["bias"],
                            p["r0"], p["pad"])
        n, T, qb, r0, rows = g["n"], g["T"], g["qb"], g["r0"], g["rows"]
        say("gemm random", p)
        q, d = hip_quantize(hip, g["x"], T, n, qb, n)
        q2, d2 = ol.quantize(g["x"], T, n, qb, n)
        assert np.array_equal(q, q2) and same(d, d2)
        want = g["out0"].copy()
        ol.gemm_q8(want, g["os"], g["w"], g["ws"], g["bias"], rows - r0, q, d, n, qb, T, g["add"], r0=r0)
        out = g["out0"].copy()
        with hip.Q8Matrix(g["w"], g["ws"]):
            bias = g["bias"][r0:] if g["bias"] is not None else None
            hip.gemm_q8(out, g["os"], g["w"], g["ws"][r0:], bias, rows - r0, hip.make_act(q, d, n, qb, T),
                        g["add"], w_offset=r0 * n, out_offset=r0)
        assert same(out, want), p


def test_quantize_random_against_oracle(hip):
    for p in cases.quant_random_params(80, seed=777):
        x = cases.quant_case(p["seed"] + 70000, p["T"], p["n"], p["qb"], p["xs"], p["scale"], p["zero_block"])
        say("quantize random", p)
        q, d = hip_quantize(hip, x, p["T"], p["n"], p["qb"], p["xs"])
        q2, d2 = ol.quantize(x, p["T"], p["n"], p["qb"], p["xs"])
        assert np.array_equal(q, q2) and same(d, d2), p
    # odd block sizes: qb = 96 (neither the column nor 16 x a power of two)
    for T, n, qb in ((3, 192, 96), (5, 480, 160), (2, 16384, 16384), (3, 8192, 8192), (4, 2048, 2048)):
        x = synth.Counter(n + qb).awkward(T * n, 3.0)
        say("quantize odd", T, n, qb)
        q, d = hip_quantize(hip, x, T, n, qb, n)
        q2, d2 = ol.quantize(x, T, n, qb, n)
        assert np.array_equal(q, q2) and same(d, d2), (T, n, qb)


def test_q8check_edges(hip):
    """tests/q8check.c:131-161: the extreme and cancelling sums, zero and
    negative scales, os 35 with the gap floats untouched, wide inputs."""
    for (n, qb, T, f) in cases.q8check_params():
        g = cases.q8check_case(n, qb, T, f)
        say("q8check", n, qb, T, f)
        want = g["out0"].copy()
        ol.gemm_q8(want, g["os"], g["w"], g["ws"], g["bias"], g["rows"], g["q"], g["d"], n, qb, T, g["add"])
        out = g["out0"].copy()
        with hip.Q8Matrix(g["w"], g["ws"]):
            hip.gemm_q8(out, g["os"], g["w"], g["ws"], g["bias"], g["rows"],
                        hip.make_act(g["q"], g["d"], n, qb, T), g["add"])
        assert same(out, want), (n, qb, T, f)


def test_no_columns_reads_and_writes_nothing(hip):
    """tests/q8check.c:156-160: T = 0 reads nothing and writes nothing."""
    out = np.array([-0.0], np.float32)
    a = hip.make_act(0, 0, 32, 32, 0)
    w = np.zeros(16 * 32, np.int8)
    ws = np.zeros(16, np.float32)
    with hip.Q8Matrix(w, ws):
        hip.gemm_q8(out, 16, w, ws, None, 16, a, 0)
    assert bits(out)[0] == 0x80000000
    hip.quantize(a, np.zeros(1, np.float32), 32)


FE = {1: 0x800, 2: 0x400, 3: 0xC00}


@pytest.mark.parametrize("rmode", [1, 2, 3])
def test_rounding_modes(hip, rmode):
    """tests/q8check.c:146-155: gemm_q8 under the three directed roundings,
    the mode read from the calling thread as the reference's ref follows it."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    for (n, qb, T, f) in [(128, 32, 5, 0), (128, 64, 5, 3), (128, 32, 37, 0), (128, 64, 37, 3),
                          (128, 128, 9, 3), (1024, 1024, 20, 1)]:
        g = cases.q8check_case(n, qb, T, f)
        say("rounding", rmode, n, qb, T, f)
        with hip.Q8Matrix(g["w"], g["ws"]):
            want, out = g["out0"].copy(), g["out0"].copy()
            a = hip.make_act(g["q"], g["d"], n, qb, T)
            assert libm.fesetround(FE[rmode]) == 0
            try:
                ol.gemm_q8(want, g["os"], g["w"], g["ws"], g["bias"], g["rows"], g["q"], g["d"], n, qb, T, g["add"])
                hip.gemm_q8(out, g["os"], g["w"], g["ws"], g["bias"], g["rows"], a, g["add"])
            finally:
                libm.fesetround(0)
        assert same(out, want), (rmode, n, qb, T, f)


@pytest.mark.parametrize("rmode", [1, 2, 3])
def test_quantize_rounding_modes(hip, rmode):
    """The table's quantize under the calling thread's directed rounding, as
    ref follows it (backend/ref/kernels.c:24-58: amax / 127, 127 / amax,
    v * id and rintf all in the mode): the oracle's bits, itself pinned to
    ref's under each mode, on the edge inputs of cases.quant_directed_cases
    (subnormal scales, products under 1/2 and on .5, rint 128 upward wrapped
    to -128, NaN and infinite blocks, xs > n)."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    for (x, T, n, qb, xs) in cases.quant_directed_cases():
        say("quantize rounding", rmode, T, n, qb, xs)
        assert libm.fesetround(FE[rmode]) == 0
        try:
            wq, wd = ol.quantize(x, T, n, qb, xs)
            q, d = hip_quantize(hip, x, T, n, qb, xs)
        finally:
            libm.fesetround(0)
        assert hip.last_kernel() == "quant_directed"
        assert np.array_equal(q, wq) and same(d, wd), (rmode, T, n, qb, xs)


def test_upload_rejects_overlapping_bytes(hip):
    """The registry is keyed on host bytes, so an upload whose bytes share any
    byte with an uploaded matrix is refused: one that contains it whole, one
    that starts inside it, one that ends inside it; a disjoint one is taken."""
    buf = np.zeros(64 * 64, np.int8)
    s16, s64 = np.ones(16, np.float32), np.ones(64, np.float32)
    with hip.Q8Matrix(buf[16 * 64:32 * 64], s16):
        for view, sc in ((buf, s64), (buf[20 * 64:36 * 64], s16), (buf[4 * 64:20 * 64], s16)):
            with pytest.raises(hip.PkHipError) as e:
                hip.Q8Matrix(view, sc)
            assert e.value.code == hip.PK_HIP_EINVAL
        with hip.Q8Matrix(buf[32 * 64:48 * 64], s16):
            pass
    with hip.Q8Matrix(buf, s64):
        pass


def test_upload_from_threads_takes_one(hip):
    """Eight threads upload the same host bytes at once: exactly one upload
    is taken and the others are refused, so no device copy is left behind
    unreachable; the one taken releases."""
    import threading
    buf = np.ones(64 * 256, np.int8)
    sc = np.ones(64, np.float32)
    taken, refused, errs = [], [], []
    start = threading.Barrier(8)

    def up():
        start.wait()
        try:
            taken.append(hip.Q8Matrix(buf, sc))
        except hip.PkHipError as e:
            (refused if e.code == hip.PK_HIP_EINVAL else errs).append(e)

    ts = [threading.Thread(target=up) for _ in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs and len(taken) == 1 and len(refused) == 7
    taken[0].release()
    with hip.Q8Matrix(buf, sc):
        pass


# --------------------------------------------- the measured shapes, whole ---

def test_single_product_full_size(hip):
    """One FastConformer feed-forward up-projection at a minute of audio:
    M = 750 frames, K = 1024 -> N = 4096, per-row quantization; every byte of
    q, d and out against the oracle."""
    g = synth.rng(0)
    M, K, N = 750, 1024, 4096
    x = synth.activations(g, M, K).reshape(-1)
    wr = synth.weights(g, N, K)
    w = synth.pack_q8(wr)
    ws = synth.scales(g, N)
    say("full size", M, K, N)
    q, d = hip_quantize(hip, x, M, K, K, K)
    q2, d2 = ol.quantize(x, M, K, K, K)
    assert np.array_equal(q, q2) and same(d, d2)
    want = np.zeros(M * N, np.float32)
    ol.gemm_q8(want, N, w, ws, None, N, q, d, K, K, M, 0, threads=16)
    out = np.zeros(M * N, np.float32)
    with hip.Q8Matrix(w, ws):
        hip.gemm_q8(out, N, w, ws, None, N, hip.make_act(q, d, K, K, M), 0)
        say("kernel", hip.last_kernel())
    assert same(out, want)


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("K,N,real", [(1024, 4096, 4096), (4096, 1024, 1024), (640, 1040, 1030), (16384, 64, 64),
                                      (4160, 32, 32)])
def test_skinny_shapes(hip, M, K, N, real):
    """Streaming shapes: M <= 16 rows. The joint's 1030 outputs are padded to
    1040 with zero rows and zero scales, as the model file pads them. K =
    16384 gives each wave several batches of units; 4160 a last batch the
    waves share unevenly."""
    g = synth.rng(M * 7 + K)
    wr = synth.weights(g, N, K)
    ws = synth.scales(g, N)
    wr[real:] = 0
    ws[real:] = 0
    w = synth.pack_q8(wr)
    x = synth.activations(g, M, K).reshape(-1)
    bias = g.standard_normal(N).astype(np.float32)
    q, d = ol.quantize(x, M, K, K, K)
    for add, use_bias in ((0, False), (1, True)):
        os_ = 0 if M == 1 else N + 3
        base = g.standard_normal(max(1, M * os_ + N)).astype(np.float32)
        want, out = base.copy(), base.copy()
        b = bias if use_bias else None
        say("skinny", M, K, N, add)
        ol.gemm_q8(want, os_, w, ws, b, N, q, d, K, K, M, add)
        with hip.Q8Matrix(w, ws):
            hip.gemm_q8(out, os_, w, ws, b, N, hip.make_act(q, d, K, K, M), add)
        assert same(out, want), (M, K, N, add)


def test_split_invariance_and_threads(hip):
    """Every output is one call's whole (core/passes.c:1-6): a product cut
    into runs of panels and chunks of columns, called from eight threads at
    once as the reference's pool calls it, gives the bits of one call."""
    g = synth.rng(5)
    M, K, N = 300, 1024, 1024
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    x = synth.activations(g, M, K).reshape(-1)
    q, d = ol.quantize(x, M, K, K, K)
    whole = np.zeros(M * N, np.float32)
    ol.gemm_q8(whole, N, w, ws, None, N, q, d, K, K, M, 0, threads=16)
    out = np.zeros(M * N, np.float32)
    items = [(r0, c0) for r0 in range(0, N, 256) for c0 in range(0, M, 48)]
    errors = []
    with hip.Q8Matrix(w, ws):
        def work(mine):
            try:
                for r0, c0 in mine:
                    nc = min(48, M - c0)
                    sub = hip.make_act(q.ctypes.data + c0 * K, d.ctypes.data + 4 * c0, K, K, nc)
                    hip.gemm_q8(out, N, w, ws[r0:], None, 256, sub, 0, w_offset=r0 * K,
                                out_offset=c0 * N + r0)
            except Exception as e:       # noqa: BLE001
                errors.append(e)
        say("threads", len(items))
        th = [threading.Thread(target=work, args=(items[i::8],)) for i in range(8)]
        for t in th:
            t.start()
        for t in th:
            t.join()
    assert not errors, errors
    assert same(out, whole)


def test_host_staging(hip):
    """The host-pointer pair moves data through two pinned 4 MiB slots: inputs
    and outputs of several slots' worth, with pitches (xs > n, os > rows),
    add's read of out, and scales other than the uploaded ones (copied per
    call) all give the oracle's bits."""
    g = synth.rng(77)
    M, K, N = 2400, 960, 1040         # x 9.2 MB, out 10 MB: three slots each, rows split across slots
    xs, os_ = K + 8, N + 5
    x = g.standard_normal(M * xs).astype(np.float32)
    say("staging quantize", M, K, xs)
    q, d = hip_quantize(hip, x, M, K, K, xs)
    q2, d2 = ol.quantize(x, M, K, K, xs)
    assert np.array_equal(q, q2) and same(d, d2)
    w = synth.pack_q8(synth.weights(g, N, K))
    ws = synth.scales(g, N)
    other = (ws * np.float32(1.5)).astype(np.float32)
    bias = g.standard_normal(N).astype(np.float32)
    base = g.standard_normal(M * os_).astype(np.float32)
    with hip.Q8Matrix(w, ws):
        for scales, add in ((ws, 1), (other, 0), (other, 1)):
            want, out = base.copy(), base.copy()
            ol.gemm_q8(want, os_, w, scales, bias, N, q, d, K, K, M, add, threads=16)
            say("staging gemm", add, scales is ws)
            hip.gemm_q8(out, os_, w, scales, bias, N, hip.make_act(q, d, K, K, M), add)
            assert same(out, want), (add, scales is ws)


def test_every_tiling(hip):
    """Every tiling of the per-column product, forced, on shapes that leave
    partial tiles in both directions, odd panel counts, K not a multiple of
    64 and a run of panels from the middle; bit for bit against the oracle."""
    shapes = [(750, 1024, 4096), (37, 96, 1040), (300, 640, 208), (129, 4096, 64), (1499, 1024, 1024), (17, 32, 16)]
    try:
        for ti in range(hip.tilings()):
            hip.force_tiling(ti)
            for (M, K, N) in shapes:
                g = synth.rng(M + K + N)
                w = synth.pack_q8(synth.weights(g, N, K))
                ws = synth.scales(g, N)
                bias = g.standard_normal(N).astype(np.float32)
                x = synth.activations(g, M, K).reshape(-1)
                q, d = ol.quantize(x, M, K, K, K)
                r0 = 16 if N > 32 else 0
                rows = N - r0
                os_ = N + 4
                base = g.standard_normal(M * os_).astype(np.float32)
                for add in (0, 1):
                    want, out = base.copy(), base.copy()
                    ol.gemm_q8(want, os_, w, ws, bias, rows, q, d, K, K, M, add, r0=r0, threads=16)
                    say("tiling", ti, M, K, N, add)
                    with hip.Q8Matrix(w, ws):
                        hip.gemm_q8(out, os_, w, ws[r0:], bias[r0:], rows, hip.make_act(q, d, K, K, M), add,
                                    w_offset=r0 * K, out_offset=r0)
                        if M > 16:
                            assert hip.last_kernel().startswith(("ring", "pipe", "stream")), hip.last_kernel()
                    assert same(out, want), (ti, M, K, N, add)
    finally:
        hip.force_tiling(-1)


def test_every_tiling_on_seeded_random_shapes(hip):
    """30 shapes drawn from a fixed seed (frames 1 to 2600, inputs 32 to
    4096 including ones that are not a multiple of 64, outputs 16 to 4096
    including 1040), with bias, add or not, output strides with and without
    padding (os = 0 at one frame), a run of panels from the middle, under the
    heuristic and every tiling forced: the oracle's bits."""
    rng = np.random.default_rng(7)
    names = [hip.tiling_name(i) for i in range(hip.tilings())]
    try:
        for case in range(30):
            M = int(rng.choice([1, 3, 16, 17, 100, 333, 750, 1201, 2600]))
            K = int(rng.choice([32, 64, 96, 320, 640, 1024, 1056, 2048, 4096]))
            N = int(rng.choice([16, 48, 208, 1024, 1040, 2048, 4096]))
            add = int(rng.integers(0, 2))
            pad = int(rng.choice([0, 1, 4]))
            r0 = 16 if N > 32 and rng.integers(0, 2) else 0
            g = synth.rng(case * 7919 + M + K + N)
            w = synth.pack_q8(synth.weights(g, N, K))
            ws = synth.scales(g, N)
            bias = g.standard_normal(N).astype(np.float32)
            x = synth.activations(g, M, K).reshape(-1)
            q, d = ol.quantize(x, M, K, K, K)
            os_ = 0 if M == 1 else N + pad
            rows = N - r0
            base = g.standard_normal(max(1, M * os_ + N)).astype(np.float32)
            want = base.copy()
            ol.gemm_q8(want, os_, w, ws, bias, rows, q, d, K, K, M, add, r0=r0, threads=16)
            with hip.Q8Matrix(w, ws):
                for ti in [-1] + list(range(hip.tilings())):
                    hip.force_tiling(ti)
                    out = base.copy()
                    say("random shape", case, M, K, N, add, pad, r0, names[ti] if ti >= 0 else "heuristic")
                    hip.gemm_q8(out, os_, w, ws[r0:], bias[r0:], rows, hip.make_act(q, d, K, K, M), add,
                                w_offset=r0 * K, out_offset=r0)
                    assert same(out, want), (case, M, K, N, add, pad, r0, hip.last_kernel())
    finally:
        hip.force_tiling(-1)
