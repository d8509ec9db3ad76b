"""The oracle, pinned (CPU only, no GPU).

The oracle (oracle/pk_oracle.c) is what the HIP path is checked against, so
it is held here to things that do not come from its own code:
  - the golden fixtures, the reference's own compiled ref backend's outputs;
  - the reference's backends themselves (oracle/_ref), where built;
  - exact rational arithmetic for the fused multiply-add and the epilogue;
  - an int64 brute force and closed forms for the integer sums;
  - the quantizer's invariants.
"""
import ctypes
import ctypes.util

import numpy as np
import pytest

import cases
import fpexact
import oracle_lib as ol
from libpktito_amd import synth


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


# ------------------------------------------------------------ fixtures ---

def test_golden_inputs_regenerate():
    man, _, _ = cases.golden()
    qc = {c[0]: c for c in cases.golden_quant_cases()}
    for m in man["quant"]:
        assert cases.digest(qc[m["name"]][1]) == m["x"], m["name"]
    gc = {g["name"]: g for g in cases.golden_gemm_cases()}
    assert len(gc) == len(man["gemm"])
    for m in man["gemm"]:
        g = gc[m["name"]]
        assert cases.digest(g["w"], g["ws"], g["bias"], g.get("x"), g["out0"]) == m["inputs"], m["name"]


def test_oracle_quantize_matches_reference_fixtures():
    man, qz, _ = cases.golden()
    for name, x, T, n, qb, xs in cases.golden_quant_cases():
        q, d = ol.quantize(x, T, n, qb, xs)
        assert np.array_equal(q, qz[f"{name}_q"]), name
        assert np.array_equal(bits(d), bits(qz[f"{name}_d"])), name


def test_oracle_gemm_matches_reference_fixtures():
    man, _, gz = cases.golden()
    acts = {m["name"]: m["act"] for m in man["gemm"]}
    for g in cases.golden_gemm_cases():
        n, T, qb = g["n"], g["T"], g["qb"]
        if "q" not in g:
            g["q"], g["d"] = ol.quantize(g["x"], T, n, qb, n)
        assert cases.digest(g["q"], g["d"]) == acts[g["name"]], g["name"]
        out = g["out0"].copy()
        ol.gemm_q8(out, g["os"], g["w"], g["ws"], g["bias"], g["rows"] - g["r0"], g["q"], g["d"],
                   n, qb, T, g["add"], r0=g["r0"])
        assert np.array_equal(bits(out), bits(gz[g["name"]])), g["name"]


# ------------------------------------------- against the reference itself ---

needs_ref = pytest.mark.skipif(ol.ref() is None, reason="oracle/_ref not built (no reference checkout)")


@needs_ref
@pytest.mark.parametrize("impl", ["ref", "avx512-vnni", "avx2-vnni", "avx2"])
def test_oracle_equals_reference_backends(impl):
    i = ol.ref_index(impl)
    if i < 0 or not ol.ref().pkref_usable(i):
        pytest.skip(f"{impl} not usable on this CPU")
    for p in cases.quant_random_params(40, seed=900):
        x = cases.quant_case(p["seed"] + 50000, p["T"], p["n"], p["qb"], p["xs"], p["scale"], p["zero_block"])
        q1, d1 = ol.quantize(x, p["T"], p["n"], p["qb"], p["xs"])
        q2, d2 = ol.quantize(x, p["T"], p["n"], p["qb"], p["xs"], impl=impl)
        assert np.array_equal(q1, q2) and np.array_equal(bits(d1), bits(d2)), p
    for p in cases.gemm_random_params(40, seed=901):
        g = cases.gemm_case(p["seed"] + 50000, p["rows"], p["n"], p["T"], p["qb"], p["add"], p["bias"],
                            p["r0"], p["pad"])
        q, d = ol.quantize(g["x"], g["T"], g["n"], g["qb"], g["n"], impl="ref")
        o1, o2 = g["out0"].copy(), g["out0"].copy()
        rows = g["rows"] - g["r0"]
        ol.gemm_q8(o1, g["os"], g["w"], g["ws"], g["bias"], rows, q, d, g["n"], g["qb"], g["T"], g["add"], r0=g["r0"])
        ol.gemm_q8(o2, g["os"], g["w"], g["ws"], g["bias"], rows, q, d, g["n"], g["qb"], g["T"], g["add"],
                   impl=impl, r0=g["r0"])
        assert np.array_equal(bits(o1), bits(o2)), p


FE = {"upward": 0x800, "downward": 0x400, "towardzero": 0xC00}


@needs_ref
@pytest.mark.parametrize("mode", ["upward", "downward", "towardzero"])
def test_oracle_follows_rounding_mode_like_ref(mode):
    """q8check's three non-default roundings (tests/q8check.c:146-155)."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    for (n, qb, T, f) in [(128, 32, 5, 0), (128, 64, 5, 3), (128, 32, 37, 0), (128, 64, 37, 3), (128, 128, 9, 3)]:
        g = cases.q8check_case(n, qb, T, f)
        o1, o2 = g["out0"].copy(), g["out0"].copy()
        assert libm.fesetround(FE[mode]) == 0
        try:
            ol.gemm_q8(o1, g["os"], g["w"], g["ws"], g["bias"], g["rows"], g["q"], g["d"], n, qb, T, g["add"])
            ol.gemm_q8(o2, g["os"], g["w"], g["ws"], g["bias"], g["rows"], g["q"], g["d"], n, qb, T, g["add"],
                       impl="ref")
        finally:
            libm.fesetround(0)
        assert np.array_equal(bits(o1), bits(o2)), (mode, n, qb, T, f)


@needs_ref
@pytest.mark.parametrize("mode", ["upward", "downward", "towardzero"])
def test_oracle_quantize_follows_rounding_mode_like_ref(mode):
    """The quantizer under each directed mode: ref follows the host's mode in
    both divisions, the product and rintf (backend/ref/kernels.c:24-58), and
    so does the oracle's restatement, bit for bit on the edge inputs (and
    unlike the nearest mode on many of them)."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    moved = 0
    for (x, T, n, qb, xs) in cases.quant_directed_cases():
        qn, dn = ol.quantize(x, T, n, qb, xs)
        assert libm.fesetround(FE[mode]) == 0
        try:
            q1, d1 = ol.quantize(x, T, n, qb, xs)
            q2, d2 = ol.quantize(x, T, n, qb, xs, impl="ref")
        finally:
            libm.fesetround(0)
        assert np.array_equal(q1, q2) and np.array_equal(bits(d1), bits(d2)), (mode, T, n, qb, xs)
        moved += int((q1 != qn).sum() + (bits(d1) != bits(dn)).sum())
        if mode == "upward":
            assert (q1 == -128).any()           # rint 128 upward, wrapped as ref's conversion wraps it
    assert moved > 100


# ------------------------------------------------------- the mathematics ---

def test_fmaf_is_one_rounding():
    """pk_fmaf (core/vmath.h:61-91): a*b+c rounded once; checked exactly."""
    o = ol.oracle()
    c = synth.Counter(77)
    a = c.uniform(4000, -1e3, 1e3)
    b = c.uniform(4000, -1e-3, 1e-3)
    cc = c.uniform(4000, -1.0, 1.0)
    specials = [(-5.0, 0.0, 0.0), (5.0, -0.0, 0.0), (-5.0, 0.0, -0.0), (3.0, 1e-40, 0.0),
                (1.0 + 2 ** -23, 1.0 - 2 ** -24, -1.0), (2 ** 100, 2 ** 100, -1.0), (1e-30, 1e-30, 0.0)]
    pairs = list(zip(a, b, cc)) + [tuple(np.float32(v) for v in s) for s in specials]
    for x, y, z in pairs:
        got = np.float32(o.pko_fmaf(x, y, z))
        want = fpexact.fma(x, y, z)
        assert bits(np.array([got]))[0] == bits(np.array([want]))[0], (x, y, z, got, want)


def test_plus_zero_addend_matters():
    """fmaf(s, 0, +0) with s < 0 is +0, where s * 0 is -0: the d = 0 blocks
    of tests/q8check.c:111-112. The oracle keeps the +0 addend."""
    T, n, rows = 1, 32, 16
    q = np.full(n, -127, np.int8)
    d = np.zeros(1, np.float32)
    w = synth.pack_q8(np.full((rows, n), 127, np.int8))
    ws = np.ones(rows, np.float32)
    out = np.full(rows, 7.0, np.float32)
    ol.gemm_q8(out, rows, w, ws, None, rows, q, d, n, n, T, 0)
    assert not np.signbit(out).any() and (out == 0).all()


def test_int_sums_against_int64_and_closed_forms():
    """kcheck's definition (tests/kcheck.c:217-239) and q8check's extremes."""
    for p in cases.gemm_random_params(20, seed=333):
        g = cases.gemm_case(p["seed"] + 7000, p["rows"], p["n"], min(p["T"], 4), p["qb"], 0, p["bias"], 0, 0)
        T = min(p["T"], 4)
        q, d = ol.quantize(g["x"], T, g["n"], g["qb"], g["n"])
        out = np.zeros(T * g["rows"], np.float32)
        ol.gemm_q8(out, g["rows"], g["w"], g["ws"], g["bias"], g["rows"], q, d, g["n"], g["qb"], T, 0)
        want = ol.definition(g["w"], g["ws"], g["bias"], g["rows"], q, d, g["n"], g["qb"], T)
        assert np.array_equal(bits(out), bits(want)), p
    # extreme sums: rows of -128 or 127 against +-127 over n = 16384
    n, rows = 16384, 16
    wr = np.empty((rows, n), np.int8)
    wr[0::2] = -128
    wr[1::2] = 127
    w = synth.pack_q8(wr)
    q = np.full(n, 127, np.int8)
    d = np.array([1.0 / 127], np.float32)
    ws = np.ones(rows, np.float32)
    out = np.zeros(rows, np.float32)
    ol.gemm_q8(out, rows, w, ws, None, rows, q, d, n, n, 1, 0)
    for r in range(rows):
        s = (-128 if r % 2 == 0 else 127) * 127 * n
        assert out[r] == fpexact.epilogue([s], [d[0]], ws[r]), r


def test_epilogue_against_exact_arithmetic():
    """The whole per-output chain, blocks of 32, with bias and add, in each
    rounding mode, against exact rationals (no libm anywhere)."""
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    modes = [(0, 0), (0x800, fpexact.UPWARD), (0x400, fpexact.DOWNWARD), (0xC00, fpexact.TOWARDZERO)]
    g = cases.gemm_case(4242, 32, 128, 3, 32, 1, 1, 0, 0)
    q, d = ol.quantize(g["x"], 3, 128, 32, 128)
    wr = synth.unpack_q8(g["w"], 32, 128).astype(np.int64)
    qq = q.reshape(3, 128).astype(np.int64)
    for fe, mode in modes:
        out = g["out0"].copy()
        assert libm.fesetround(fe) == 0
        try:
            ol.gemm_q8(out, g["os"], g["w"], g["ws"], g["bias"], 32, q, d, 128, 32, 3, 1)
        finally:
            libm.fesetround(0)
        for t in range(3):
            for r in range(32):
                sums = [int((wr[r, b * 32:(b + 1) * 32] * qq[t, b * 32:(b + 1) * 32]).sum()) for b in range(4)]
                want = fpexact.epilogue(sums, d[t * 4:(t + 1) * 4], g["ws"][r], g["bias"][r],
                                        g["out0"][t * g["os"] + r], mode)
                got = out[t * g["os"] + r]
                assert bits(np.array([got]))[0] == bits(np.array([want]))[0], (mode, t, r, got, want)


def test_quantizer_invariants():
    """q in [-127, 127], never -128; a zero block exactly when it holds a NaN,
    an infinity, or amax < 2^-121; d = amax / 127 and q = rint(x * (127 /
    amax)), each a single float32 rounding (numpy's float32 ops are IEEE)."""
    x, T, n, qb, top = cases.quant_tiny()
    q, d = ol.quantize(x, T, n, qb, n)
    for t in range(T):
        for b in range(n // qb):
            assert (d[t * (n // qb) + b] == 0) == (top[b] < np.float32(2.0 ** -121))
    x, T, n, qb = cases.quant_nonfinite()
    q, d = ol.quantize(x, T, n, qb, n)
    assert (q == 0).all() and (d == 0).all() and not np.signbit(d).any()
    for p in cases.quant_random_params(30, seed=5150):
        x = cases.quant_case(p["seed"], p["T"], p["n"], p["qb"], p["xs"], p["scale"], p["zero_block"])
        q, d = ol.quantize(x, p["T"], p["n"], p["qb"], p["xs"])
        assert q.min() >= -127
        n, qb = p["n"], p["qb"]
        for t in range(p["T"]):
            for b in range(n // qb):
                v = x[t * p["xs"] + b * qb: t * p["xs"] + (b + 1) * qb]
                amax = np.float32(np.abs(v).max())
                qq = q[t * n + b * qb: t * n + (b + 1) * qb]
                dd = d[t * (n // qb) + b]
                if amax < np.float32(2.0 ** -121):
                    assert dd == 0 and (qq == 0).all()
                    continue
                assert dd == np.float32(amax / np.float32(127.0))
                idv = np.float32(127.0) / amax
                assert np.array_equal(qq, np.rint((v * idv).astype(np.float32)).astype(np.int8))


def test_pk_q8_index_and_packing_agree():
    o = ol.oracle()
    c = synth.Counter(31)
    rows, n = 48, 96
    w = c.int8(rows * n).reshape(rows, n)
    p = synth.pack_q8(w)
    for r in range(0, rows, 7):
        for k in range(0, n, 5):
            assert p[o.pko_q8_index(n, r, k)] == w[r, k]
    assert np.array_equal(synth.unpack_q8(p, rows, n), w)
