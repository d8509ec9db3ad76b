"""The int8 product path on one MI355X: encoder-GEMM milliseconds per audio
minute over the 24-layer FastConformer encoder's int8 products at ten
minutes of audio, with the roofline of its dominant kernel and the same
workload on the host's cores beside it.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--quick] [--no-cpu]

A step is one pass of the hot path over one batch: the 24 layers' int8
products (each layer's q, k, v, o, the positions' projection on 2M - 1
rows, the two feed-forward modules' 1024 -> 4096 and 4096 -> 1024, the
convolution module's pointwise 1024 -> 2048 and 1024 -> 1024, d_model
1024, 8 heads) at M = 7500 frames, every layer with independent weights
(~0.6 GB of int8 resident in HBM), each product's input the previous one's
fp32 output quantized per row to int8, multiplied with exact int32 sums into
fp32 outputs by the reference's epilogue. Weights, scales and the first fp32
input are synthetic (int8 uniform [-127, 127], scales uniform [1e-3, 1e-2]
scaled so the chain stays finite, N(0, 1) frames) and resident in HBM before
the timed region. A sweep's 385 launches (a quantize and a product each,
q, k, v and the positions in one launch) are captured once into a HIP graph
and replayed; K replays are timed with events on the stream they run on.
`value` is the sweep's milliseconds over its ten minutes of audio.

`roofline` is the dominant kernel's (the product kernel taking the most
time a layer), timed alone in a graph of back-to-back launches. `cpu_baseline`
runs the same chain, on the same weights and input, with the reference's
fastest kernels this host runs (compiled from its sources into oracle/_ref)
over every core. The `extra` object adds the sweep's TOPS and per-product
kernels, the sweep at one minute of audio, one layer's products at M = 750
(per-row and in the encoder's blocks of 32 and 64), the device-resident
layer (the whole of core/encoder.c's layer in HBM) beside the same layer on
the host's cores, the long-form layer and a ragged batch of 8 segments in
grouped launches, the skinny (M <= 16) shapes against HBM, the decoder's
token steps and the host-pointer drop-in as the reference's pool deals it.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_INT8_PEAK_TOPS = 5000.0      # MI355X dense int8, published
HBM_PEAK_GBS = 8000.0             # MI355X HBM3E, published


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--quick", action="store_true", help="the headline sweep only: no extras, no CPU baseline")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--profile-kernel", default=None,
                   help="only launch the named product's kernel 50 times (for rocprofv3 --pmc runs)")
    p.add_argument("--profile-layer", type=int, default=0, metavar="QB",
                   help="only replay the device-resident layer at M=750 in blocks of QB (for rocprofv3)")
    p.add_argument("--profile-m", type=int, default=750, metavar="M",
                   help="frames of --profile-kernel's product (750 or 7500)")
    p.add_argument("--profile-sweep", type=int, default=0, metavar="M",
                   help="only replay the 24-layer sweep at M frames --steps times (for rocprofv3)")
    p.add_argument("--profile-skinny", default=None, metavar="M,K,N",
                   help="only M-row products through rotated K x N matrices, 50 launches (for rocprofv3)")
    p.add_argument("--profile-decoder", action="store_true",
                   help="the decoder's token steps only (graphs of a prediction and a joint, no CPU leg)")
    p.add_argument("--profile-step", action="store_true",
                   help="only the per-row layer step at one minute of audio, its graph replayed --steps times")
    p.add_argument("--peaks", action="store_true",
                   help="only the on-machine check of the int8 MFMA and HBM read peaks")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only copy 256 MiB three times (the known-size kernel that scales "
                        "rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


# --------------------------------------------------------------- device ---

class Product:
    """One int8 product of the layer, resident in HBM: its uploaded matrix, its
    fp32 input, its quantized activations (row-major q, d, and the packed copy
    the product reads) and its fp32 output."""

    def __init__(self, pk, torch, name, M, K, N, half, add, g, x_dev=None, xs=None, ws_gain=1.0):
        from libpktito_amd import synth
        self.name, self.M, self.K, self.N, self.add = name, M, K, N, int(add)
        self.quantizes = True
        wr = synth.weights(g, N, K)
        self.w = synth.pack_q8(wr)
        self.ws = (synth.scales(g, N) * np.float32(ws_gain)).astype(np.float32)
        self.m = pk.Q8Matrix(self.w, self.ws)
        dev = torch.device("cuda")
        if x_dev is None:
            self.x_host = synth.activations(g, M, K, half)
            self.x = torch.from_numpy(self.x_host).to(dev)
            self.xs = K
        else:
            self.x_host = None
            self.x, self.xs = x_dev, xs
        self.q = torch.empty((M, K), dtype=torch.int8, device=dev)
        self.d = torch.empty((M,), dtype=torch.float32, device=dev)
        self.qp = torch.empty((pk.packed_bytes(K, M),), dtype=torch.int8, device=dev)
        self.out = torch.zeros((M, N), dtype=torch.float32, device=dev)

    def share(self, other):
        """Take other's quantized activations as this product's input (the
        reference multiplies q, k and v by one quantized activation)."""
        self.quantizes = False
        self.x_host, self.x, self.q, self.d, self.qp = other.x_host, other.x, other.q, other.d, other.qp

    def ops(self):
        return 2.0 * self.M * self.K * self.N

    def gemm_bytes(self):
        M, K, N = self.M, self.K, self.N
        return N * K + 4 * N + M * K + 4 * M + 4 * M * N + (4 * M * N if self.add else 0)

    def quant_bytes(self):
        return 4 * self.M * self.K + self.M * self.K + 4 * self.M

    def quantize(self, pk, stream=None, packed=True):
        if packed:
            # the products read the packed copy only: no row-major q is written
            pk.quantize_packed_dev(None, self.qp, self.d, self.x, self.K, self.M, self.xs, stream=stream)
        else:
            pk.quantize_dev(self.q, self.d, self.x, self.K, self.K, self.M, self.xs, stream=stream)

    def gemm(self, pk, stream=None, packed=True):
        if packed:
            pk.gemm_q8_packed_dev(self.out, self.N, self.m, 0, self.N, self.m.dev_scales, None, self.qp, self.d,
                                  self.K, self.M, self.add, stream=stream)
        else:
            pk.gemm_q8_dev(self.out, self.N, self.m, 0, self.N, None, None, self.q, self.d, self.K, self.K,
                           self.M, self.add, ws_ptr=self.m.dev_scales, stream=stream)


def make_layer(pk, torch, M, seed, ws_gain=None):
    """One layer's products in the reference's dataflow (core/encoder.c:329-368):
    k and v multiply q's quantized activation; the positions' projection reads
    positional encodings quantized once an encode (core/encoder.c:467-469), so
    its quantize is done here, outside the layer step."""
    from libpktito_amd import synth
    g = synth.rng(seed)
    prods = []
    for (name, mm, K, N, half, add) in synth.layer_products(M):
        gain = 1.0 if ws_gain is None else ws_gain(K)
        prods.append(Product(pk, torch, name, mm, K, N, half, add, g, ws_gain=gain))
    by = {p.name: p for p in prods}
    by["k"].share(by["q"])
    by["v"].share(by["q"])
    by["pos"].quantize(pk)
    by["pos"].quantizes = False
    torch.cuda.synchronize()
    return prods


def graph_of(torch, fn):
    """fn's launches captured into a HIP graph on a side stream."""
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()        # once outside capture, so every lazy set-up has happened
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps, warmup):
    """ms per replay of graph g: warmup replays, then reps replays between two
    events on the current stream, synchronized on both sides."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def kernel_ms(pk, torch, prod, launches=64, reps=5, packed=True):
    """The average duration of one product's kernel: a graph of `launches`
    back-to-back launches of it, timed with events on its stream."""
    def fn():
        for _ in range(launches):
            prod.gemm(pk, packed=packed)
    g = graph_of(torch, fn)
    best = min(time_graph(torch, g, 3, 1) for _ in range(reps))
    return best / launches


# ------------------------------------------------------------ workloads ---

ATTENTION = ("q", "k", "v", "pos")


def batch_gemm(pk, group, stream=None):
    """The attention's independent products (q, k, v of one activation and the
    positions' projection) in one launch."""
    pk.gemm_q8_batch_dev([(p.out, p.N, p.m, 0, p.N, p.m.dev_scales, None, p.qp, p.d, p.K, p.M, p.add)
                          for p in group], stream=stream)


def layer_step(pk, prods, packed=True, batch=True):
    """One layer's quantizes and products in the reference's order; with batch,
    q, k, v and pos go to one launch after q's quantize."""
    group = [p for p in prods if p.name in ATTENTION] if batch and packed else []

    def fn():
        for p in prods:
            if group and p.name in ATTENTION:
                if p is group[0]:
                    for a in group:
                        if a.quantizes:
                            a.quantize(pk)
                    batch_gemm(pk, group)
                continue
            if p.quantizes:
                p.quantize(pk, packed=packed)
            p.gemm(pk, packed=packed)
    return fn


def check_replay(pk, torch, prods, graph):
    """A replay's outputs equal an eager step's, bit for bit (graphs replayed
    several times with eager work between)."""
    fn = layer_step(pk, prods)
    for _ in range(3):
        for p in prods:
            p.out.zero_()
        fn()
        torch.cuda.synchronize()
        eager = [p.out.clone() for p in prods]
        for p in prods:
            p.out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for p, e in zip(prods, eager):
            if not torch.equal(p.out.view(torch.int32), e.view(torch.int32)):
                return False
    return True


def encoder_sweep(pk, torch, M, seed):
    """The 24-layer encoder's products: with independent weights (~0.6 GB of int8 in HBM),
    each product's input the previous product's fp32 output re-quantized per
    row, in the order ff1_up, ff1_down, q (k and v multiply q's activation and
    go to one launch with the positions' projection), o (on v's output), pw1
    (first 1024 of its 2048 columns into pw2), pw2, ff2_up, ff2_down; the
    positions' projection reads the positional encodings, quantized once an
    encode as the reference does.
    Each matrix's scales are the configs' uniform [1e-3, 1e-2] times
    1 / (sqrt(K) * 73.6 * 0.0055) so that a chain of 264 products keeps its
    activations finite (timing does not depend on the values)."""
    from libpktito_amd import synth
    dev = torch.device("cuda")
    g = synth.rng(seed)
    x0 = torch.from_numpy(synth.activations(g, M, 1024)).to(dev)
    ape = torch.from_numpy(synth.activations(g, 2 * M - 1, 1024)).to(dev)
    ape_q = torch.empty((2 * M - 1, 1024), dtype=torch.int8, device=dev)
    ape_d = torch.empty((2 * M - 1,), dtype=torch.float32, device=dev)
    ape_qp = torch.empty((pk.packed_bytes(1024, 2 * M - 1),), dtype=torch.int8, device=dev)
    gain = lambda K: 1.0 / (np.sqrt(K) * 73.6 * 0.0055)   # noqa: E731
    order = ["ff1_up", "ff1_down", "q", "k", "v", "o", "pw1", "pw2", "ff2_up", "ff2_down"]
    shapes = {p[0]: p for p in synth.layer_products(M)}
    layers = []
    prev = x0
    prev_xs = 1024
    for L in range(24):
        lay = {}
        for name in order:
            _, mm, K, N, half, add = shapes[name]
            p = Product(pk, torch, name, mm, K, N, half, add, g, x_dev=prev, xs=prev_xs, ws_gain=gain(K))
            if name in ("k", "v"):
                p.share(lay["q"])           # one activation for q, k and v, as the reference has
            lay[name] = p
            if name not in ("q", "k"):
                prev, prev_xs = p.out, N
        _, mm, K, N, half, add = shapes["pos"]
        pp = Product(pk, torch, "pos", mm, K, N, half, add, g, x_dev=ape, xs=1024, ws_gain=gain(K))
        pp.q, pp.d, pp.qp = ape_q, ape_d, ape_qp
        lay["pos"] = pp
        layers.append(lay)
        prev = lay["ff2_down"].out
        prev_xs = 1024

    def fn():
        pk.quantize_packed_dev(ape_q, ape_qp, ape_d, ape, 1024, 2 * M - 1, 1024)
        for lay in layers:
            for name in order[:2]:
                lay[name].quantize(pk)
                lay[name].gemm(pk)
            lay["q"].quantize(pk)
            batch_gemm(pk, [lay[n] for n in ATTENTION])
            for name in order[5:]:
                p = lay[name]
                p.quantize(pk)
                p.gemm(pk)
    ops = sum(p.ops() for lay in layers for p in lay.values())
    return fn, ops, layers


def skinny_rates(pk, torch, shapes, budget_bytes=640 << 20, rows=(1, 4, 16), launches=None):
    """Skinny products: M in {1, 4, 16} rows through weights rotated over more than
    512 MB of distinct matrices, so that L2 and the 256 MB MALL serve none of
    them. One graph of launches over the copies; GB/s from the algorithmic
    bytes N K + 4 N + M K + 4 M + 4 M N of each launch. Beside each, the
    floors it is read against, in graphs of as many launches: an empty
    kernel, and a streaming read of the same bytes through a rotation of the
    same size (of_stream_read: the read's time over the product's)."""
    from libpktito_amd import synth
    dev = torch.device("cuda")
    out = []
    for (K, N, real) in shapes:
        per = N * K
        copies = max(8, budget_bytes // per + 1)
        g = synth.rng(K * 31 + N)
        big = g.integers(-127, 128, size=copies * per, dtype=np.int8)
        wsa = synth.scales(g, N)
        mats = []
        for c in range(copies):
            wslice = big[c * per:(c + 1) * per]
            mats.append(pk.Q8Matrix(wslice, wsa))
        rot = torch.empty((copies * per + 64 * 1024,), dtype=torch.uint8, device=dev)
        rot.random_(0, 256)
        sink = torch.zeros((4,), dtype=torch.int32, device=dev)
        for M in rows:
            x = torch.from_numpy(synth.activations(g, M, K)).to(dev)
            q = torch.empty((M, K), dtype=torch.int8, device=dev)
            d = torch.empty((M,), dtype=torch.float32, device=dev)
            pk.quantize_dev(q, d, x, K, K, M, K)
            o = torch.empty((M, N), dtype=torch.float32, device=dev)
            # the split over K's workspace, zero, shared by the rotation's
            # launches (one stream: they run one after another)
            work = torch.zeros((pk.gemm_workspace(N),), dtype=torch.uint8, device=dev)

            if launches:
                # eager launches over the rotation, for a counter run
                for i in range(launches):
                    m = mats[i % len(mats)]
                    pk.gemm_q8_dev(o, N, m, 0, N, None, None, q, d, K, K, M, 0, ws_ptr=m.dev_scales, work=work)
                torch.cuda.synchronize()
                out.append(dict(M=M, K=K, N=N, launches=launches, kernel=pk.last_kernel(),
                                bytes_per_launch=N * K + 4 * N + M * K + 4 * M + 4 * M * N))
                continue

            def fn():
                for m in mats:
                    pk.gemm_q8_dev(o, N, m, 0, N, None, None, q, d, K, K, M, 0, ws_ptr=m.dev_scales, work=work)
            gr = graph_of(torch, fn)
            ms = min(time_graph(torch, gr, 2, 1) for _ in range(3)) / len(mats)
            kname = pk.last_kernel()
            byts = N * K + 4 * N + M * K + 4 * M + 4 * M * N
            # the yardsticks: the same number of back-to-back launches of an
            # empty kernel, and of a streaming read of the same bytes through
            # a rotation of the same size
            rd = (byts + 15) // 16 * 16

            def read():
                for c in range(len(mats)):
                    pk.stream_read_dev(rot[c * per:], sink, nbytes=rd)
            gs = graph_of(torch, read)
            rms = min(time_graph(torch, gs, 2, 1) for _ in range(3)) / len(mats)
            ge = graph_of(torch, lambda: [pk.empty_dev() for _ in mats])
            ems = min(time_graph(torch, ge, 2, 1) for _ in range(3)) / len(mats)
            del gr, gs, ge
            out.append(dict(M=M, K=K, N=N, outputs=real, us=round(ms * 1e3, 3),
                            GBs=round(byts / (ms * 1e-3) / 1e9, 1),
                            hbm_frac=round(byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 3),
                            stream_read_us=round(rms * 1e3, 3), empty_launch_us=round(ems * 1e3, 3),
                            of_stream_read=round(rms / ms, 3), kernel=kname))
        for m in mats:
            m.release()
        del big, rot
    return out


def peak_check(pk, torch):
    """The two published peaks the rooflines divide by, checked on this
    machine: the int8 matrix cores' rate (2048 workgroups of four waves, each
    wave 4096 rounds of eight independent 16x16x64 MFMAs on registers, 32768
    ops an MFMA), and a streaming read of 4 GiB (ten times the 256 MB MALL).
    Each is the best of three launches timed with events on the current
    stream, the stream the launches go to."""
    sink = torch.zeros((4,), dtype=torch.int32, device="cuda")
    wgs, iters = 2048, 4096
    ops = wgs * 4 * iters * 8 * 32768

    def best(fn):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        return min(ts)
    mms = best(lambda: pk.mfma_rate_dev(wgs, iters, sink))
    buf = torch.empty((4 << 30,), dtype=torch.uint8, device="cuda")
    buf.random_(0, 256)
    rms = best(lambda: pk.stream_read_dev(buf, sink))
    del buf
    torch.cuda.empty_cache()
    tops = ops / (mms * 1e-3) / 1e12
    gbs = (4 << 30) / (rms * 1e-3) / 1e9
    return dict(mfma_int8_tops=round(tops, 1), of_published_mfma=round(tops / MFMA_INT8_PEAK_TOPS, 3),
                hbm_read_GBs=round(gbs, 1), of_published_hbm=round(gbs / HBM_PEAK_GBS, 3),
                mfma_ms=round(mms, 3), read_ms=round(rms, 3))


# --------------------------------------------------------- CPU baseline ---

def cpu_impls():
    """The host's kernels to time, fastest first: the reference's SIMD
    backends this CPU can run and its scalar ref (compiled from its sources
    into oracle/_ref), or the oracle's C restatement when that is absent.
    Each is (kind, backend id, quantize(act, x_ptr, xs), gemm(out_ptr, os,
    w_ptr, ws_ptr, rows, act, add)), both dealt over `cores` threads as the
    reference's pool deals them (core/passes.c:28-46, :80-109)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol
    cores = min(os.cpu_count() or 1, 64)
    out = []
    if ol.ref() is not None:
        r = ol.ref()
        for bid in ("avx512-vnni", "avx2-vnni", "ref"):
            i = ol.ref_index(bid)
            if i >= 0 and r.pkref_usable(i):
                out.append(("reference", bid,
                            lambda a, x, xs, i=i: r.pkref_quantize_threads(i, cores, ctypes.byref(a), x, xs),
                            lambda o, os_, w, ws, rows, a, add, i=i: r.pkref_gemm_threads(
                                i, cores, o, os_, w, ws, None, rows, ctypes.byref(a), add)))
    if not out:
        o = ol.oracle()
        fq = ctypes.cast(o.pko_quantize, ctypes.c_void_p).value
        fg = ctypes.cast(o.pko_gemm_q8, ctypes.c_void_p).value
        out.append(("port", "oracle",
                    lambda a, x, xs: o.pko_quantize_threads(fq, cores, ctypes.byref(a), x, xs),
                    lambda op, os_, w, ws, rows, a, add: o.pko_gemm_threads(fg, cores, op, os_, w, ws, None, rows,
                                                                           ctypes.byref(a), add)))
    return cores, out


def cpu_sweep(layers, M, seconds, impl, frames=None):
    """The chained sweep on this host's cores: encoder_sweep's order, weights
    and inputs (its first layer's input and the positional encodings copied
    from the device), each product's input quantized per row from the
    previous product's fp32 output (pw2 on the first 1024 of pw1's 2048
    floats a frame, xs = 2048), the positions quantized once an encode. Layer
    after layer of the chain, pass after pass over the 24, until `seconds`
    have gone by (at least one layer), then the time a layer times 24. Every
    step works frame by frame, so with `frames` F < M the chain runs the
    first F frames (and 2F - 1 positions) alone and the time is per F
    frames; ms per audio-minute is the time over F / 750 minutes."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol
    kind, bid, quant, gemm = impl
    F = M if frames is None else min(frames, M)
    R = 2 * F - 1
    x0 = np.ascontiguousarray(layers[0]["ff1_up"].x[:F].cpu().numpy())
    ape = np.ascontiguousarray(layers[0]["pos"].x[:R].cpu().numpy())
    bufs = {}

    def buf(name, shape, dtype=np.float32):
        if name not in bufs:
            bufs[name] = np.zeros(shape, dtype)
        return bufs[name]

    def act(x, xs, K, T, tag):
        q = buf("q" + tag, (T * K,), np.int8)
        d = buf("d" + tag, (T,))
        a = ol.Act(q.ctypes.data, d.ctypes.data, K, K, T)
        quant(a, x.ctypes.data, xs)
        return a

    def run(p, a, T):
        out = buf(p.name, (T, p.N))
        gemm(out.ctypes.data, p.N, p.w.ctypes.data, p.ws.ctypes.data, p.N, a, p.add)
        return out

    def layers_of_the_chain():
        """The chain's layers one by one, pass after pass over the 24."""
        while True:
            pa = act(ape, 1024, 1024, R, "pos")        # once an encode
            x = x0
            for lay in layers:
                h = run(lay["ff1_up"], act(x, 1024, 1024, F, "a"), F)
                fd = run(lay["ff1_down"], act(h, 4096, 4096, F, "b"), F)
                a = act(fd, 1024, 1024, F, "a")
                for n in ("q", "k", "v"):
                    run(lay[n], a, F)
                run(lay["pos"], pa, R)
                o = run(lay["o"], act(bufs["v"], 1024, 1024, F, "a"), F)
                p1 = run(lay["pw1"], act(o, 1024, 1024, F, "a"), F)
                p2 = run(lay["pw2"], act(p1, 2048, 1024, F, "a"), F)
                u = run(lay["ff2_up"], act(p2, 1024, 1024, F, "a"), F)
                x = run(lay["ff2_down"], act(u, 4096, 4096, F, "b"), F)
                yield

    t0 = time.perf_counter()
    done = 0
    for _ in layers_of_the_chain():
        done += 1
        if time.perf_counter() - t0 >= seconds:
            break
    el = time.perf_counter() - t0
    return dict(kind=kind, backend=bid, ms_per_audio_minute=el / done * 24 * 1e3 / (F / 750.0), layers=done,
                frames=F, seconds=round(el, 2))


def cpu_baseline(prods_host, seconds):
    """The reference's backends on this host's cores, on the layer's inputs:
    each product quantized per row (16 frames an item) and multiplied in
    64-row slices dealt from an atomic counter over every core
    (tests/gemmbench.c:77-94, core/passes.c:28-46 in the reference)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol
    cores = min(os.cpu_count() or 1, 64)
    impls = []
    if ol.ref() is not None:
        for bid in ("avx512-vnni", "avx2-vnni", "ref"):
            i = ol.ref_index(bid)
            if i >= 0 and ol.ref().pkref_usable(i):
                impls.append(("reference", bid, i))
    if not impls:
        impls.append(("port", "oracle", -1))
    results = {}
    for kind, bid, idx in impls[:1] + [x for x in impls[1:] if x[1] == "ref"]:
        bufs = []
        for (x, w, ws, M, K, N, add) in prods_host:
            q = np.zeros(M * K, np.int8)
            d = np.zeros(M, np.float32)
            out = np.zeros(M * N, np.float32)
            bufs.append((x, w, ws, M, K, N, add, q, d, out))
        lim = seconds if bid != "ref" else seconds / 2
        # the scalar ref takes ~1.5 s a layer on 16 cores: a quarter of the layer's frames
        frac = 1.0 if bid != "ref" else 0.25
        reps, ops, t0 = 0, 0.0, time.perf_counter()
        while True:
            for (x, w, ws, M, K, N, add, q, d, out) in bufs:
                Ms = max(1, int(M * frac))
                a = ol.Act(q.ctypes.data, d.ctypes.data, K, K, Ms)
                if idx >= 0:
                    ol.ref().pkref_quantize_threads(idx, cores, ctypes.byref(a), x.ctypes.data, K)
                    ol.ref().pkref_gemm_threads(idx, cores, out.ctypes.data, N, w.ctypes.data, ws.ctypes.data,
                                                None, N, ctypes.byref(a), add)
                else:
                    o = ol.oracle()
                    fq = ctypes.cast(o.pko_quantize, ctypes.c_void_p).value
                    fg = ctypes.cast(o.pko_gemm_q8, ctypes.c_void_p).value
                    o.pko_quantize_threads(fq, cores, ctypes.byref(a), x.ctypes.data, K)
                    o.pko_gemm_threads(fg, cores, out.ctypes.data, N, w.ctypes.data, ws.ctypes.data, None, N,
                                       ctypes.byref(a), add)
                ops += 2.0 * Ms * K * N
            reps += 1
            el = time.perf_counter() - t0
            if el >= lim:
                break
        results[bid] = dict(kind=kind, tops=ops / el / 1e12, reps=reps, seconds=el, cores=cores, frac=frac)
    return results


def device_layer(pk, torch, M, qb, reps=20, warmup=3):
    """The device-resident encoder layer (core/encoder.c:321-368: its eleven
    int8 products, the fused producers and the attention's float part) at M
    frames in blocks of qb, one pk_hip_layer_dev call captured in a HIP graph
    and replayed on the same x. Returns (us a layer, the weights and host
    inputs for a CPU leg)."""
    from libpktito_amd import synth
    g = synth.rng(77 + qb)
    w = synth.layer_weights(g, D=1024, H=8, F=4096, K=9)
    x = g.standard_normal((M, 1024)).astype(np.float32)
    ape = g.standard_normal((2 * M - 1, 1024)).astype(np.float32)
    lay = pk.DeviceLayer(w, torch)
    R = 2 * M - 1
    ape_qp = torch.zeros((pk.packed_bytes(1024, R),), dtype=torch.int8, device="cuda")
    ape_d = torch.empty((R * (1024 // qb),), dtype=torch.float32, device="cuda")
    pk.quantize_packed_dev(None, ape_qp, ape_d, torch.from_numpy(ape).cuda(), 1024, R, 1024, qb=qb)
    ws = torch.empty((lay.workspace(M, qb),), dtype=torch.uint8, device="cuda")
    xt = torch.from_numpy(x).cuda()
    gph = graph_of(torch, lambda: lay.run(xt, M, ape_qp, ape_d, qb, ws))
    ms = time_graph(torch, gph, reps, warmup)
    lay.release()
    del gph
    return ms * 1e3, (w, x, ape)


def decoder_steps(pk, torch, with_cpu, cpu_seconds=2.0):
    """The decoder's token steps (core/decoder.c:54-101) at the model's shapes
    (pred_hidden 640, 2 LSTM layers, joint 640, vocabulary 1024 + blank, 5
    durations): a prediction (one token's L + 1 launches) and a joint (two
    launches) each captured in a HIP graph and replayed; the joint with the
    readback of its token and duration that a host-driven search needs each
    step; and the same steps on one host core from the reference's fastest
    kernels (the reference splits only products of 2048 rows or more, over
    at most 4 threads)."""
    from libpktito_amd import synth
    dec = synth.decoder_weights(synth.rng(90))
    dd = pk.DeviceDecoder(dec, torch)
    J = dec["J"]
    f = torch.from_numpy((synth.rng(91).standard_normal(J) * 2).astype(np.float32)).cuda()
    out = {}
    gp = graph_of(torch, lambda: dd.predict(5))
    out["predict_us"] = round(time_graph(torch, gp, 200, 10) * 1e3, 2)
    gj = graph_of(torch, lambda: dd.joint(f))
    out["joint_us"] = round(time_graph(torch, gj, 200, 10) * 1e3, 2)
    reps = 200
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        dd.joint(f)
        dd.tok_dur.cpu()
    out["joint_with_readback_us"] = round((time.perf_counter() - t0) / reps * 1e6, 2)
    out["launches"] = dict(predict=dec["L"] + 1, joint=2)
    # the whole search in one launch (pk_hip_search_dev) over a minute of
    # frames (750), synthetic frames at two scales (the larger emits more
    # tokens); the call returns with the tokens on the host
    V, blank, durs = dec["V"], dec["V"], [0, 1, 2, 3, 4]
    T = 750
    searches = []
    for scale in (1.0, 2.0):
        frames = (synth.rng(92).standard_normal((T, J)) * scale).astype(np.float32)
        fd = torch.from_numpy(frames).cuda()
        toks = dd.search(fd, T, blank, durs, 10)
        reps = 5
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            dd.search(fd, T, blank, durs, 10)
        ms = (time.perf_counter() - t0) / reps * 1e3
        searches.append(dict(frames=T, scale=scale, tokens=len(toks), ms=round(ms, 3),
                             us_per_frame=round(ms * 1e3 / T, 2), frames_host=frames, dev_toks=toks))
    dd.release()
    del gp, gj
    if with_cpu:
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as ol
        impl = "oracle"
        if ol.ref() is not None:
            for bid in ("avx512-vnni", "avx2-vnni"):
                i = ol.ref_index(bid)
                if i >= 0 and ol.ref().pkref_usable(i):
                    impl = bid
                    break
        dw = ol.DecoderWeights(dec)
        h = np.zeros((dec["L"], dec["P"]), np.float32)
        c = np.zeros_like(h)
        fh = f.cpu().numpy()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds / 2:
            h, c, g = ol.predict(dw, 5, h, c, impl=impl)
            n += 1
        tp = (time.perf_counter() - t0) / n
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds / 2:
            ol.joint(dw, fh, g, impl=impl)
            n += 1
        tj = (time.perf_counter() - t0) / n
        out["cpu_1_thread"] = dict(backend=impl, predict_us=round(tp * 1e6, 2), joint_us=round(tj * 1e6, 2),
                                   kind="reference" if impl != "oracle" else "port")
        # the same searches on one host thread: their joints and predictions
        # counted by running the search on the oracle's steps, each costed at
        # the times above
        from tdt_search import search as tdt
        for sr in searches:
            frames = sr["frames_host"]
            cnt = {"j": 0, "p": 0}
            st = {"h": np.zeros((dec["L"], dec["P"]), np.float32), "c": np.zeros((dec["L"], dec["P"]), np.float32),
                  "gp": None}

            def o_predict(k):
                cnt["p"] += 1
                st["h"], st["c"], st["gp"] = ol.predict(dw, k, st["h"], st["c"])

            def o_joint(t):
                cnt["j"] += 1
                _, k, di = ol.joint(dw, frames[t], st["gp"])
                return k, di
            toks = tdt(T, o_predict, o_joint, blank, durs, 10)
            sr["same_tokens_as_oracle_search"] = toks == sr["dev_toks"]
            sr["joints"], sr["predictions"] = cnt["j"], cnt["p"]
            sr["cpu_1_thread_ms"] = round((cnt["j"] * tj + cnt["p"] * tp) * 1e3, 3)
    for sr in searches:
        sr.pop("frames_host")
        sr.pop("dev_toks")
    out["search_one_launch"] = searches
    return out


def cpu_layer(w, x, ape, M, qb, seconds):
    """The same layer on this host's cores from the reference's fastest
    usable backend's own kernels (oracle/_ref), composed in core/encoder.c's
    order and dealt over every core in the reference's items (the oracle's
    composition, pinned to give the oracle's bits with them)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol
    cores = min(os.cpu_count() or 1, 64)
    impl, kind = "oracle", "port"
    if ol.ref() is not None:
        for bid in ("avx512-vnni", "avx2-vnni"):
            i = ol.ref_index(bid)
            if i >= 0 and ol.ref().pkref_usable(i):
                impl, kind = bid, "reference"
                break
    R = 2 * M - 1
    ape_q, ape_d = ol.quantize(ape.reshape(-1), R, 1024, qb, 1024)
    reps, t0 = 0, time.perf_counter()
    while True:
        ol.conformer_layer(w, x, M, ape_q, ape_d, qb, threads=cores, impl=impl)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return dict(ms_per_layer=round(el / reps * 1e3, 2), layers=reps, seconds=round(el, 1), cores=cores,
                kind=kind, backend=impl)


def recorded_traffic(kernel, M, K, N):
    """HBM bytes a launch of this kernel on this shape, as the rocprofv3
    FETCH_SIZE / WRITE_SIZE passes summarized under profiles/ measured them
    (each scaled by the same counter on a copy of known size); None when no
    summary covers this kernel and shape."""
    import glob
    import re
    want = f"kernel={kernel} M={M} K={K} N={N} "
    for f in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.txt"))):
        with open(f) as fh:
            for line in fh:
                if line.startswith("pmc: ") and want in line:
                    m = re.search(r"traffic_bytes=(\d+)", line)
                    if m:
                        return int(m.group(1))
    return None


def copy_calibration(torch):
    """A plain copy of 256 MiB, three times: the known-size kernel whose
    rocprofv3 FETCH_SIZE and WRITE_SIZE scale a product's to bytes."""
    a = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    return {"copied_bytes": a.numel() * 4, "times": 3}


def reference_pool(threads=16, seconds=1.0):
    """The reference's own pool entries timed by its library (oracle/_ref's
    dropin_cli --time-passes: pk_quantize_on then pk_gemm_on, 750 x 1024 ->
    4096, THREADS pool threads, host pointers, PCIe inside each hip call),
    unchanged (dropin_cli: 47 quantize items of 16 frames, 64-row slices of
    the product) and with the core/passes.c change (dropin_cli_whole: one
    call each under hip), on the hip table and on avx512-vnni."""
    import subprocess
    out = {}
    for prog, key in (("dropin_cli", "pool_dealing"), ("dropin_cli_whole", "whole_product_change")):
        path = os.path.join(ROOT, "oracle", "_ref", prog)
        if not os.path.exists(path):
            out[key] = "absent (the reference checkout was absent when the oracle was built)"
            continue
        res = {}
        for table in ("hip", "avx512-vnni"):
            env = dict(os.environ, PKTITO_KERNELS=table)
            r = subprocess.run([path, "--time-passes", str(threads), str(seconds)], capture_output=True, text=True,
                               env=env, timeout=300)
            if r.returncode != 0:
                res[table] = f"failed: {r.stderr.strip()[-300:]}"
                continue
            d = json.loads(r.stdout.strip().splitlines()[-1])
            res[table] = dict(quantize_us=round(d["quantize_ms"] * 1e3, 1), gemm_q8_us=round(d["gemm_ms"] * 1e3, 1),
                              tops=round(d["tops"], 2), calls=d["calls"], threads=d["threads"],
                              table=d["table"].split(" (")[0], check=d["check"])
        out[key] = res
    out["note"] = ("host pointers through the reference's pool (core/passes.c), the hip table staging each call's "
                   "activations and outputs over PCIe; the same outputs (check) on every table and dealing")
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ------------------------------------------------------------------ main ---

SWEEP_M = 7500          # ten minutes of audio in one segment


def dominant(pk, torch, prods, launches, reps):
    """Each product's kernel alone (kernel_ms: a graph of back-to-back
    launches, HIP events on its stream), grouped by kernel and shape (ff1 and
    ff2 share theirs); the group taking the most time a layer is the
    dominant kernel. Returns (per product, the dominant group's product,
    its kernel's name, its us a launch)."""
    per, groups = {}, {}
    for p in prods:
        kms = kernel_ms(pk, torch, p, launches=launches, reps=reps)
        kname = pk.last_kernel()
        per[p.name] = dict(us=round(kms * 1e3, 2), kernel=kname, tops=round(p.ops() / (kms * 1e-3) / 1e12, 1),
                           GBs=round(p.gemm_bytes() / (kms * 1e-3) / 1e9, 1),
                           pct_mfma=round(100 * p.ops() / (kms * 1e-3) / 1e12 / MFMA_INT8_PEAK_TOPS, 1))
        key = (kname, p.M, p.K, p.N, p.add)
        tot, _, _ = groups.get(key, (0.0, p, kms))
        groups[key] = (tot + kms, p, kms)
    _, dom, dkms = max(groups.values(), key=lambda t: t[0])
    return per, dom, per[dom.name]["kernel"], dkms


def roofline_of(dom, dname, dkms):
    dbytes = dom.gemm_bytes()
    intensity = dom.ops() / dbytes
    bound = "hbm" if intensity < MFMA_INT8_PEAK_TOPS * 1e12 / (HBM_PEAK_GBS * 1e9) else "mfma"
    r = dict(bound=bound, kernel=dname, product=f"{dom.name} M={dom.M} K={dom.K} N={dom.N}",
             unit="GB/s" if bound == "hbm" else "TFLOP/s",
             achieved=round(dbytes / (dkms * 1e-3) / 1e9 if bound == "hbm" else dom.ops() / (dkms * 1e-3) / 1e12, 1),
             peak=HBM_PEAK_GBS if bound == "hbm" else MFMA_INT8_PEAK_TOPS,
             kernel_us=round(dkms * 1e3, 3), bytes_per_launch=dbytes, ops_per_launch=dom.ops(),
             traffic=recorded_traffic(dname, dom.M, dom.K, dom.N))
    r["frac"] = round(r["achieved"] / r["peak"], 4)
    # achieved and frac count the algorithmic (minimum) bytes a launch; the
    # same launch's profiled HBM traffic, where a summary covers it, gives
    # the rate the memory actually moved, named apart
    if bound == "hbm" and r["traffic"]:
        r["achieved_traffic"] = round(r["traffic"] / (dkms * 1e-3) / 1e9, 1)
        r["frac_traffic"] = round(r["achieved_traffic"] / r["peak"], 4)
    return r


def release(layers):
    for lay in layers:
        for p in lay.values():
            p.m.release()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not run "
              "(the int8 path would shard frames across GPUs with no exchange)", file=sys.stderr)
        sys.exit(2)
    import torch
    if args.copy_calibration:
        print(json.dumps(copy_calibration(torch)))
        return
    import libpktito_amd as pk
    pk.init()
    torch.cuda.set_device(0)

    M = 750
    if args.peaks:
        print(json.dumps({"peaks_measured": peak_check(pk, torch)}))
        return
    if args.profile_decoder:
        print(json.dumps({"profiled": "decoder_steps", **decoder_steps(pk, torch, False)}))
        return
    if args.profile_step:
        prods = make_layer(pk, torch, M, seed=1)
        graph = graph_of(torch, layer_step(pk, prods))
        ms = time_graph(torch, graph, args.steps, args.warmup)
        print(json.dumps({"profiled": "layer_step", "M": M, "replays": args.steps, "ms_per_step": round(ms, 5)}))
        return
    if args.profile_layer:
        us, _ = device_layer(pk, torch, M, args.profile_layer, reps=args.steps, warmup=args.warmup)
        print(json.dumps({"profiled": "device_layer", "M": M, "qb": args.profile_layer, "us_per_layer": round(us, 1),
                          "replays": args.steps}))
        return
    if args.profile_sweep:
        fn, _, layers = encoder_sweep(pk, torch, args.profile_sweep, seed=10 + args.profile_sweep)
        gs = graph_of(torch, fn)
        ms = time_graph(torch, gs, args.steps, args.warmup)
        print(json.dumps({"profiled": "encoder_sweep", "M": args.profile_sweep, "replays": args.steps,
                          "ms_per_sweep": round(ms, 3)}))
        return
    if args.profile_skinny:
        Ms, Ks, Ns = (int(v) for v in args.profile_skinny.split(","))
        r = skinny_rates(pk, torch, [(Ks, Ns, Ns)], rows=(Ms,), launches=50)
        print(json.dumps({"profiled": "skinny", **r[0], "calibration": copy_calibration(torch)}))
        return
    if args.profile_kernel:
        # the named product's kernel alone, 50 times: what the rocprofv3
        # summaries under profiles/ are cut from
        prods = make_layer(pk, torch, args.profile_m, seed=1 if args.profile_m == 750 else 2)
        dom = next(p for p in prods if p.name == args.profile_kernel)
        for _ in range(50):
            dom.gemm(pk)
        torch.cuda.synchronize()
        kname = pk.last_kernel()
        for p in prods:
            p.m.release()
        del prods
        torch.cuda.empty_cache()
        # the known-size copy in the same process, so one counter run scales both
        print(json.dumps({"profiled": dom.name, "M": dom.M, "kernel": kname, "launches": 50,
                          "bytes_per_launch": dom.gemm_bytes(), "ops_per_launch": dom.ops(),
                          "calibration": copy_calibration(torch)}))
        return

    # ---- the headline: the 24-layer chained sweep at ten minutes of audio
    fn, sops, layers = encoder_sweep(pk, torch, SWEEP_M, seed=10 + SWEEP_M)
    gs = graph_of(torch, fn)
    log(f"sweep M={SWEEP_M} captured")
    ms = time_graph(torch, gs, args.steps, args.warmup)
    minutes = SWEEP_M / 750.0
    value = ms / minutes
    tops = sops / (ms * 1e-3) / 1e12
    log(f"sweep M={SWEEP_M}: {ms:.3f} ms, {value:.4f} ms per audio-minute, {tops:.1f} TOPS")
    del gs
    first = [layers[0][n] for n in ("ff1_up", "ff1_down", "q", "k", "v", "pos", "o", "pw1", "pw2", "ff2_up",
                                    "ff2_down")]
    per_long, dom, dname, dkms = dominant(pk, torch, first, launches=8, reps=3)
    roofline = roofline_of(dom, dname, dkms)
    log(f"dominant {dom.name}: {dkms * 1e3:.2f} us ({dname})")
    extra = dict(sweep_M7500=dict(ms_per_sweep=round(ms, 3), tops=round(tops, 1),
                                  pct_mfma_peak=round(100 * tops / MFMA_INT8_PEAK_TOPS, 2), ops_per_sweep=sops,
                                  per_product_first_layer=per_long))
    cpu = None
    if not args.no_cpu and not args.quick:
        cores, impls = cpu_impls()
        cpu = cpu_sweep(layers, SWEEP_M, args.cpu_seconds, impls[0])
        cpu["cores"] = cores
        log(f"cpu sweep: {cpu}")
        scalar = [i for i in impls[1:] if i[1] == "ref"]
        if scalar:
            r = cpu_sweep(layers, SWEEP_M, args.cpu_seconds / 2, scalar[0], frames=750)
            r["cores"] = cores
            extra["cpu_ref_scalar_sweep"] = r
    release(layers)
    del layers, fn
    torch.cuda.empty_cache()

    if not args.quick:
        extra["peaks_measured"] = peak_check(pk, torch)
        log(f"peaks: {extra['peaks_measured']}")

    if not args.quick:
        # the same sweep at one minute of audio
        fn, sops750, layers = encoder_sweep(pk, torch, M, seed=10 + M)
        gs = graph_of(torch, fn)
        sms = time_graph(torch, gs, 20, 3)
        log(f"sweep M={M}: {sms:.3f} ms")
        extra["sweep_M750"] = dict(ms_per_sweep=round(sms, 3), ms_per_audio_minute=round(sms, 4),
                                   tops=round(sops750 / (sms * 1e-3) / 1e12, 1),
                                   pct_mfma_peak=round(100 * sops750 / (sms * 1e-3) / 1e12 / MFMA_INT8_PEAK_TOPS, 2))
        release(layers)
        del layers, gs, fn
        torch.cuda.empty_cache()

    if not args.quick:
        # ---- one layer's products at one minute of audio, per-row, one graph a step
        prods = make_layer(pk, torch, M, seed=1)
        step = layer_step(pk, prods)
        graph = graph_of(torch, step)
        replay_ok = check_replay(pk, torch, prods, graph)
        lms = time_graph(torch, graph, 50, 5)
        ops = sum(p.ops() for p in prods)
        ltops = ops / (lms * 1e-3) / 1e12
        per750, dom750, dname750, dkms750 = dominant(pk, torch, prods, launches=64, reps=5)
        extra["layer_M750"] = dict(ms_per_step=round(lms, 5), tops=round(ltops, 1),
                                   pct_mfma_peak=round(100 * ltops / MFMA_INT8_PEAK_TOPS, 2),
                                   graph_replay_matches_eager=replay_ok, per_product=per750,
                                   roofline=roofline_of(dom750, dname750, dkms750),
                                   layer_quantize_bytes=sum(p.quant_bytes() for p in prods),
                                   layer_gemm_bytes=sum(p.gemm_bytes() for p in prods))
        log(f"layer M=750: {lms:.4f} ms a step, {ltops:.1f} TOPS")
        host_inputs = [(p.x_host.reshape(-1), p.w, p.ws, p.M, p.K, p.N, p.add) for p in prods]

        # the real encoder's blocks (qb = 32 by default, 64 in its fast mode): the
        # same layer with blocked quantizes and products on the packed path, q, k,
        # v and pos in one launch as in the per-row step
        blocked = {}
        for qb in (32, 64):
            bd = {p.name: torch.empty((p.M * p.K // qb,), dtype=torch.float32, device=p.x.device) for p in prods}
            src = {p.name: p for p in prods}
            owner = {"k": "q", "v": "q"}
            pos = src["pos"]
            pk.quantize_packed_dev(None, pos.qp, bd["pos"], pos.x, pos.K, pos.M, pos.xs, qb=qb)  # once an encode

            def blocked_step(qb=qb, bd=bd):
                for p in prods:
                    o = src[owner.get(p.name, p.name)]
                    if p.name not in owner and p.name != "pos":
                        pk.quantize_packed_dev(None, p.qp, bd[p.name], p.x, p.K, p.M, p.xs, qb=qb)
                    if p.name in ATTENTION:
                        if p.name == ATTENTION[0]:
                            group = [(a, src[owner.get(a.name, a.name)]) for a in prods if a.name in ATTENTION]
                            pk.gemm_q8_batch_dev([(a.out, a.N, a.m, 0, a.N, a.m.dev_scales, None, ao.qp, bd[ao.name],
                                                   a.K, a.M, a.add) for a, ao in group], qb=qb)
                        continue
                    pk.gemm_q8_packed_dev(p.out, p.N, p.m, 0, p.N, p.m.dev_scales, None, o.qp, bd[o.name], p.K, p.M,
                                          p.add, qb=qb)
            gb = graph_of(torch, blocked_step)
            bms = time_graph(torch, gb, 50, 5)
            blocked[f"qb{qb}"] = dict(ms_per_step=round(bms, 4), tops=round(ops / (bms * 1e-3) / 1e12, 1),
                                      kernel=pk.last_kernel())
            log(f"layer qb={qb}: {bms:.4f} ms")
            del gb
        extra["layer_M750_blocked"] = blocked

        # the device-resident layer (the whole of core/encoder.c's layer in HBM:
        # fused layer norm, SiLU and depthwise producers, the attention's float
        # products, the eleven products), in the encoder's blocks
        dlayer = {}
        host_layer = None
        for qb in (32, 64):
            us, host = device_layer(pk, torch, M, qb)
            dlayer[f"qb{qb}"] = dict(us_per_layer=round(us, 1),
                                     encoder_ms_per_audio_minute_24_layers=round(us * 24e-3, 2),
                                     int8_product_tops=round(ops / (us * 1e-6) / 1e12, 1))
            log(f"device layer qb={qb}: {us:.1f} us")
            if qb == 32:
                host_layer = host
            torch.cuda.empty_cache()
        extra["device_layer_M750"] = dlayer

        # the long-form layer, M = 7500 (one segment of ten minutes)
        long_prods = make_layer(pk, torch, 7500, seed=2)
        gl = graph_of(torch, layer_step(pk, long_prods))
        lfms = time_graph(torch, gl, 10, 3)
        lops = sum(p.ops() for p in long_prods)
        log(f"long form: {lfms:.3f} ms a layer")
        extra["long_form_M7500"] = dict(ms_per_layer=round(lfms, 4), tops=round(lops / (lfms * 1e-3) / 1e12, 1),
                                        pct_mfma_peak=round(100 * lops / (lfms * 1e-3) / 1e12 / MFMA_INT8_PEAK_TOPS,
                                                            1))
        for p in long_prods:
            p.m.release()
        del long_prods, gl
        torch.cuda.empty_cache()

        # a ragged batch of 8 segments (12-60 s), each product one
        # grouped launch over the segments (the quantize over their rows at once)
        from libpktito_amd import synth
        lens = synth.ragged_lengths()
        rg = synth.rng(3)
        dev = torch.device("cuda")
        rag = []
        tot = sum(lens)
        offs = np.cumsum([0] + lens)
        for (name, mm, K, N, half, add) in synth.layer_products(750):
            if name == "pos":
                continue    # the positions' rows are per segment (2M - 1), not a frame batch
            p = Product(pk, torch, name, tot, K, N, half, add, rg)
            segs = [(p.out[offs[i]:offs[i + 1]], N, p.q[offs[i]:offs[i + 1]], p.d[offs[i]:offs[i + 1]],
                     K, K, lens[i]) for i in range(len(lens))]
            rag.append((p, segs))

        def rag_step():
            for p, segs in rag:
                p.quantize(pk, packed=False)
                pk.gemm_q8_grouped_dev(p.m, 0, p.N, p.m.dev_scales, None, segs, p.add)
        grg = graph_of(torch, rag_step)
        rms = time_graph(torch, grg, 20, 3)
        rops = sum(p.ops() for p, _ in rag)
        log(f"ragged: {rms:.3f} ms")
        extra["ragged_8_segments"] = dict(frames=lens, ms_per_layer_ex_pos=round(rms, 4),
                                          tops=round(rops / (rms * 1e-3) / 1e12, 1))
        for p, _ in rag:
            p.m.release()
        del rag, grg

        # skinny shapes against HBM
        extra["skinny"] = skinny_rates(pk, torch, [(1024, 4096, 4096), (4096, 1024, 1024), (640, 1040, 1030)])

        # the decoder's token steps in their own fused launches
        extra["decoder_steps"] = decoder_steps(pk, torch, not args.no_cpu)
        log("decoder steps done")

        log("skinny done")

        # the host-pointer drop-in inside the reference's own library: its
        # pool entries pk_quantize_on / pk_gemm_on on the configs' first
        # product, on the hip table and the reference's avx512-vnni, dealt
        # as the unchanged core/passes.c deals them and with the
        # whole-product change (part of the CPU-baseline leg: the programs
        # are the reference's library built under oracle/_ref)
        if not args.no_cpu:
            extra["reference_pool_ff1_up_M750"] = reference_pool()
            log("reference pool done")
        if not args.no_cpu:
            lc = cpu_baseline(host_inputs, args.cpu_seconds / 2)
            extra["layer_M750"]["cpu"] = {k: dict(tops=round(v["tops"], 4), cores=v["cores"], kind=v["kind"],
                                                  frames_frac=v["frac"], seconds=round(v["seconds"], 1))
                                          for k, v in lc.items()}
            log("cpu layer products done")
            w, x, ape = host_layer
            extra["device_layer_M750"]["cpu_qb32"] = cpu_layer(w, x, ape, M, 32, args.cpu_seconds / 2)
            log("cpu layer done")
        for p in prods:
            p.m.release()

    line = {
        "metric": "int8 GEMM TOPS (% of MFMA peak); encoder-GEMM ms per audio-minute, 1 GPU",
        "value": round(value, 4),
        "unit": "ms per audio-minute",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded int8 weights uniform [-127, 127], per-channel scales; fp32 N(0,1) input "
                "frames; random-init weights of the encoder's shapes, no checkpoint)",
        "config": {"workload": f"24-layer FastConformer encoder int8 GEMM sweep at M={SWEEP_M} frames (ten "
                               "minutes of audio, one segment): every layer's q,k,v,o, positions (2M-1 rows), "
                               "ff1/ff2 up 1024->4096 and down 4096->1024, pw1 1024->2048, pw2 1024->1024, "
                               "independent weights (~0.6 GB int8 resident), each product's input the previous "
                               "one's fp32 output quantized per row; one HIP graph a sweep",
                   "M": SWEEP_M, "layers": 24, "d_model": 1024, "ff": 4096, "qb": "per-row (n)",
                   "audio_minutes": minutes, "ops_per_step": sops, "tops": round(tops, 1),
                   "pct_mfma_peak": round(100 * tops / MFMA_INT8_PEAK_TOPS, 2)},
        "roofline": roofline,
        "cpu_baseline": None,
        "extra": extra,
    }
    if cpu:
        line["cpu_baseline"] = dict(
            value=round(cpu["ms_per_audio_minute"], 2), unit="ms per audio-minute", cores=cpu["cores"],
            kind=cpu["kind"],
            sample=f"the same sweep (same weights and input, M={cpu['frames']}) on the reference's "
                   f"{cpu['backend']} kernels dealt over {cpu['cores']} threads: {cpu['layers']} layers of the "
                   f"chain (passes over its 24) in {cpu['seconds']} s, the time a layer times 24; {cpu_model()}")
    print(json.dumps(line))


if __name__ == "__main__":
    main()
