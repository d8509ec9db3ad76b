"""The cases the parity tests run, generated from seeds so that the golden
fixtures (cut from the reference's compiled ref backend) store only the
case's parameters and the reference's outputs.

They follow the reference's own kernel tests:
  - kcheck (tests/kcheck.c:98-241, 498-532): random shapes, qb in {32, 64, n},
    add and bias, runs of panels from the middle, output strides with a gap,
    and kcheck's awkward values: +-0, subnormals, x30 outliers, ties, zero
    blocks, non-finite inputs, amax either side of 2^-121;
  - q8check (tests/q8check.c:85-161): weights of -128 and 127 against
    activations of +-127 (the extreme sums, and exact cancellation), zero
    scales, negative per-row scales, an output stride of 35, wide inputs;
and add the shapes this path is measured on (per-row qb at n = 1024, 4096, 640
with N padded from 1030 to 1040).
"""
import hashlib

import numpy as np

from libpktito_amd import synth


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()[:16]


# ------------------------------------------------------------- quantize ---

def quant_case(seed, T, n, qb, xs, scale, zero_block):
    """kcheck's quant_case: awkward values over T*xs + n floats, and (when
    zero_block) a first block of zeros."""
    c = synth.Counter(seed)
    x = c.awkward(T * xs + n, scale)
    if zero_block:
        x[:qb] = 0.0
    return x


def quant_nonfinite():
    """kcheck's quant_nonfinite_case: NaN and +-inf in some blocks."""
    T, n, qb = 2, 64, 32
    x = synth.Counter(7).uniform(T * n)
    x[3] = np.nan
    x[40] = np.inf
    x[n + 5] = -np.inf
    x[n + 45] = np.nan
    return x, T, n, qb


def quant_tiny():
    """kcheck's quant_tiny_case: blocks whose amax sits either side of 2^-121."""
    top = np.array([2.0 ** -140, 2.0 ** -130, 2.0 ** -122, float.fromhex("0x1.fffffep-122"),
                    2.0 ** -121, 2.0 ** -120, 2.0 ** -100], np.float32)
    qb, T = 32, 2
    n = qb * len(top)
    c = synth.Counter(11)
    x = np.zeros(T * n, np.float32)
    for t in range(T):
        for b, tp in enumerate(top):
            v = (tp * c.uniform(qb)).astype(np.float32)
            pick = int(c.bits(3)[0] % np.uint64(qb))
            v[pick] = -tp if t else tp
            v[2 * int(c.bits(1)[0] % np.uint64(qb // 2))] = 0.0
            v[2 * int(c.bits(1)[0] % np.uint64(qb // 2)) + 1] = -0.0
            x[t * n + b * qb: t * n + (b + 1) * qb] = v
    return x, T, n, qb, top


def quant_directed_cases(seed=300):
    """Inputs for the quantizer under directed rounding (ref follows the host's
    mode in amax / 127, 127 / amax, v * id and rintf): (x, T, n, qb, xs).
    Rows 0-6 of each carry the edges: blocks at and just above the 2^-121
    zero rule (subnormal d), a constant block (products of 127 exactly),
    small integers, a large value beside tiny, subnormal and signed-zero
    ones (products under 1/2), halves (products on .5), a NaN and an
    infinity; the rest N(0, 9), whose largest value reaches rint 128 upward."""
    out = []
    for i, (T, n, qb, pad) in enumerate([(37, 256, 32, 0), (37, 256, 64, 32), (21, 256, 256, 0), (9, 1024, 1024, 32),
                                         (5, 64, 32, 0)]):
        g = synth.rng(seed + i)
        xs = n + pad
        x = (g.standard_normal(T * xs) * 3).astype(np.float32)
        r = [x[t * xs:t * xs + n] for t in range(min(T, 7))]
        r[0][:] = np.float32(2.0 ** -121) * g.standard_normal(n).astype(np.float32)
        r[1][:] = np.float32(2.0 ** -119)
        r[2][:] = (np.arange(n) % 33 - 16).astype(np.float32)
        r[3][:] = g.uniform(-1e-3, 1e-3, n).astype(np.float32)
        r[3][::8] = np.float32(100.0)
        r[3][1::8] = np.float32(1e-40)
        r[3][2::8] = np.float32(-0.0)
        r[3][3::8] = np.float32(-1e-40)
        if len(r) > 4:
            r[4][:] = (np.arange(n) % 16 - 8).astype(np.float32) + np.float32(0.5)
            r[4][::qb] = np.float32(127.0)
        if len(r) > 5:
            r[5][qb // 2] = np.nan
        if len(r) > 6:
            r[6][(qb + 1) % n] = np.inf
        out.append((x, T, n, qb, xs))
    return out


def quant_random_params(count, seed=100):
    """kcheck's run(): n = 32 * (1 + r % 40), T in [1, 20], qb 32 or n,
    xs = n or n + 32, scale 1 or 1e4; and its fast mode's qb = 64."""
    c = synth.Counter(seed)
    out = []
    for rep in range(count):
        b = c.bits(6)
        if rep % 4 == 3:
            n = 64 * (1 + int(b[0] % np.uint64(20)))
            qb = 64
        else:
            n = 32 * (1 + int(b[0] % np.uint64(40)))
            qb = 32 if b[2] % np.uint64(2) else n
        T = 1 + int(b[1] % np.uint64(20))
        xs = n + 32 * int(b[3] % np.uint64(2))
        scale = 1.0 if rep % 3 else 1e4
        out.append(dict(seed=1000 + rep, T=T, n=n, qb=qb, xs=xs, scale=scale,
                        zero_block=bool(b[4] % np.uint64(3) == 0)))
    return out


# -------------------------------------------------------------- gemm_q8 ---

def gemm_case(seed, rows, n, T, qb, add, bias, r0, pad):
    """kcheck's gemm_q8_case: weights mostly uniform in [-127, 127] and one in
    three 127, scales 0.01 (frand + 1.5) or one in eight 0, awkward biases,
    activations awkward(2) quantized (by whoever the caller trusts), the output
    stride rows or rows + 16, and the output pre-filled with awkward(1).
    Returns a dict of inputs; 'x' is to be quantized with qb."""
    c = synth.Counter(seed)
    w_rm = np.where(c.bits(rows * n) % np.uint64(3) != 0, c.int8(rows * n), np.int8(127))
    w_rm = w_rm.astype(np.int8).reshape(rows, n)
    ws = np.where(c.bits(rows) % np.uint64(8) != 0,
                  (np.float32(0.01) * (c.uniform(rows) + np.float32(1.5))).astype(np.float32),
                  np.float32(0.0)).astype(np.float32)
    b = c.awkward(rows, 1.0)
    x = c.awkward(T * n, 2.0)
    os_ = rows + 16 * pad
    out0 = c.awkward(T * os_, 1.0)
    return dict(w=synth.pack_q8(w_rm), ws=ws, bias=b if bias else None, x=x, os=os_,
                out0=out0, rows=rows, n=n, T=T, qb=qb, add=add, r0=r0)


def gemm_random_params(count, seed=200, ns=(32, 64, 96, 256, 640, 1024, 4096)):
    """kcheck's run() and fast_cases(): n from its list, rows 16 to 384 (64 at
    n = 4096), T 1 (every fourth case) or up to 37, qb 32 / 64 / n, add and
    bias each half the time, and a run of panels from the middle."""
    c = synth.Counter(seed)
    out = []
    for rep in range(count):
        b = c.bits(9)
        n = ns[int(b[0] % np.uint64(len(ns)))]
        rows = 16 * (1 + int(b[1] % np.uint64(24)))
        T = 1 if rep % 4 == 0 else 1 + int(b[2] % np.uint64(37))
        if n == 4096 and rows > 64:
            rows = 64
        sel = int(b[3] % np.uint64(3))
        qb = n if sel == 0 else (64 if (sel == 2 and n % 64 == 0) else 32)
        add = int(b[4] % np.uint64(2))
        bias = int(b[5] % np.uint64(2))
        r0 = 16 * int(b[6] % np.uint64(rows // 16)) if rows > 16 and b[7] % np.uint64(2) else 0
        pad = int(b[8] % np.uint64(2))
        out.append(dict(seed=2000 + rep, rows=rows, n=n, T=T, qb=qb, add=add, bias=bias, r0=r0, pad=pad))
    return out


def q8check_case(n, qb, T, flags):
    """q8check's q8_case: 32 rows, os 35, rows of -128, of 127, of 127/-127 and
    of 127/-128 by turns; activations +127, -127 or alternating; block scales
    0 where (k + t) % 5 == 0 else ((k + t) % 13 + 1) / 127; per-row scales
    +-1/32; biases r % 7 - 3.25; outputs pre-filled 0.125 / -0."""
    rows, os_ = 32, 35
    nb = n // qb
    r = np.arange(rows)[:, None]
    k = np.arange(n)[None, :]
    w = np.where(r % 4 == 0, -128,
        np.where(r % 4 == 1, 127,
        np.where(r % 4 == 2, np.where(k % 2 == 1, -127, 127),
                 np.where(k % 2 == 1, -128, 127)))).astype(np.int8)
    t = np.arange(T)[:, None]
    q = np.where(t % 3 == 0, 127, np.where(t % 3 == 1, -127,
                 np.where(k % 2 == 1, -127, 127))).astype(np.int8).reshape(-1)
    kb = np.arange(nb)[None, :]
    d = np.where((kb + t) % 5 == 0, np.float32(0.0),
                 ((kb + t) % 13 + 1).astype(np.float32) / np.float32(127.0)).astype(np.float32).reshape(-1)
    ws = np.where(np.arange(rows) % 2 == 1, -0.03125, 0.03125).astype(np.float32)
    b = (np.arange(rows) % 7).astype(np.float32) - np.float32(3.25)
    out0 = np.where(np.arange(T * os_) % 2 == 1, np.float32(-0.0), np.float32(0.125)).astype(np.float32)
    return dict(w=synth.pack_q8(w), q=q, d=d, ws=ws, bias=b if flags & 1 else None, out0=out0,
                rows=rows, os=os_, n=n, qb=qb, T=T, add=(flags >> 1) & 1)


def q8check_params():
    """q8check's run(): n in {32, 64, 96, 128, 1024, 4096} x qb {32, 64} x T 1..9
    x the four flag pairs (a subset of T), both sides of a column block's edge,
    and the widest input, 16384."""
    out = []
    for n in (32, 64, 96, 128, 1024, 4096):
        for qb in sorted({32, 64, n}):
            if n % qb:
                continue
            for T in (1, 2, 5, 9):
                for f in range(4):
                    out.append((n, qb, T, f))
    for qb in (32, 64):
        out += [(4096, qb, 49, 3), (4096, qb, 50, 3), (1024, qb, 193, 3), (1024, qb, 194, 3),
                (16384, qb, 13, 3), (16384, qb, 14, 3)]
    return out


# -------------------------------------------------- the golden fixtures ---

def golden_quant_cases():
    """(name, x, T, n, qb, xs) of every quantize fixture."""
    out = []
    for p in quant_random_params(24):
        x = quant_case(p["seed"], p["T"], p["n"], p["qb"], p["xs"], p["scale"], p["zero_block"])
        out.append((f"random{p['seed']}", x, p["T"], p["n"], p["qb"], p["xs"]))
    x, T, n, qb = quant_nonfinite()
    out.append(("nonfinite", x, T, n, qb, n))
    x, T, n, qb, _ = quant_tiny()
    out.append(("tiny", x, T, n, qb, n))
    for n, T in ((1024, 6), (4096, 3), (640, 5), (16384, 2)):
        c = synth.Counter(300 + n)
        x = sum(c.uniform(T * n) for _ in range(4)).astype(np.float32)    # N(0,1)-like
        out.append((f"perrow{n}", x, T, n, n, n))
    return out


def golden_gemm_cases():
    """(name, dict) of every gemm_q8 fixture, with 'q' and 'd' quantized by ref."""
    out = []
    for p in gemm_random_params(28):
        g = gemm_case(p["seed"], p["rows"], p["n"], p["T"], p["qb"], p["add"], p["bias"],
                            p["r0"], p["pad"])
        g["name"] = f"random{p['seed']}"
        g["seed"] = p["seed"]
        g["pad"] = p["pad"]
        out.append(g)
    for (n, qb, T, f) in q8check_params():
        if n > 4096 or T > 50:
            continue
        if (n, T) in ((4096, 49), (4096, 50)) or (T == 2 and f in (1, 2)):
            continue
        g = q8check_case(n, qb, T, f)
        g["name"] = f"q8check_n{n}_qb{qb}_T{T}_f{f}"
        g["r0"] = 0
        out.append(g)
    # per-row products of the measured shapes: K=1024 -> 256 rows, K=4096 -> 64,
    # and the joint's K=640 -> 1030 outputs padded to 1040 with zero rows
    for (rows, n, T, pad_rows) in ((256, 1024, 8, 0), (64, 4096, 4, 0), (1040, 640, 1, 10),
                                   (1040, 640, 16, 10)):
        c = synth.Counter(400 + n + T)
        w = c.int8(rows * n).reshape(rows, n)
        ws = c.uniform(rows, 1e-3, 1e-2)
        if pad_rows:
            w[rows - pad_rows:] = 0
            ws[rows - pad_rows:] = 0.0
        x = sum(c.uniform(T * n) for _ in range(4)).astype(np.float32)
        out.append(dict(name=f"perrow_{rows}x{n}_T{T}", w=synth.pack_q8(w), ws=ws, bias=None, x=x,
                        os=rows, out0=np.zeros(T * rows, np.float32), rows=rows, n=n, T=T, qb=n,
                        add=0, r0=0, seed=400 + n + T))
    return out


def golden_dir():
    import os
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden():
    """(manifest, quant arrays, gemm arrays) of the committed fixtures."""
    import json
    import os
    d = golden_dir()
    with open(os.path.join(d, "manifest.json")) as f:
        man = json.load(f)
    return man, np.load(os.path.join(d, "quant.npz")), np.load(os.path.join(d, "gemm.npz"))
