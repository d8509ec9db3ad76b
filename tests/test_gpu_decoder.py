"""The decoder's token steps on the GPU against the oracle, bit for bit: the
fused gemv, an LSTM layer's step (both products, their add and the cell), the
joint's logits and argmax (including ties, signed zeros and NaNs placed by
hand), the prediction network over several tokens with its state in HBM,
and a greedy TDT search (core/decoder.c:104-140) driven the same way over
the device steps and over the oracle's, which must emit the same tokens."""
import sys

import numpy as np
import pytest

import oracle_lib as ol
from tdt_search import search
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


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.device("cuda"))


@pytest.mark.parametrize("rows,cols,add,withbias,off", [(1040, 640, 0, True, 0), (2560, 640, 0, True, 0),
                                                       (640, 640, 1, False, 0), (16, 64, 0, False, 0),
                                                       (48, 4096, 1, True, 0), (32, 1056, 0, True, 0),
                                                       (1040, 640, 0, True, 1), (32, 1056, 1, False, 3)])
def test_gemv(hip, torch, rows, cols, add, withbias, off):
    """cols 1056 takes the 64-unit kernel; off > 0 puts x off 16-byte
    alignment (the kernel's four-load rows)."""
    g = synth.rng(rows + cols + add)
    w = synth.pack_q8(synth.weights(g, rows, cols))
    ws = synth.scales(g, rows)
    x = (g.standard_normal(cols) * 2).astype(np.float32)
    bias = g.standard_normal(rows).astype(np.float32) if withbias else None
    old = g.standard_normal(rows).astype(np.float32)
    q, d = ol.quantize(x, 1, cols, cols, cols)
    want = old.copy()
    ol.gemm_q8(want, 0, w, ws, bias, rows, q, d, cols, cols, 1, add)
    out = dev(torch, old)
    say("gemv", rows, cols, add, withbias)
    with hip.Q8Matrix(w, ws) as m:
        xt = dev(torch, np.concatenate([np.zeros(off, np.float32), x]))[off:]
        hip.gemv_dev(out, m, dev(torch, bias) if bias is not None else None, xt, add)
        torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(want))


def decoder(seed, model):
    if model:
        return synth.decoder_weights(synth.rng(seed))
    return synth.decoder_weights(synth.rng(seed), P=64, L=2, J=64, V=40, n_dur=5)


@pytest.mark.parametrize("model", [False, True])
def test_predict_over_tokens(hip, torch, model):
    """The prediction network over a run of labels, its state carried in HBM,
    against the oracle's predict step by step."""
    dec = decoder(11, model)
    dw = ol.DecoderWeights(dec)
    dd = hip.DeviceDecoder(dec, torch)
    try:
        P, L = dec["P"], dec["L"]
        h = np.zeros((L, P), np.float32)
        c = np.zeros((L, P), np.float32)
        for step, label in enumerate([dec["V"] - 1, 0, 5, 5, dec["V"] - 2, 17]):
            say("predict", model, step, label)
            dd.predict(label)
            torch.cuda.synchronize()
            h, c, gp = ol.predict(dw, label, h, c)
            dh, dc = dd.state()
            assert np.array_equal(bits(dh.cpu().numpy()), bits(h)), step
            assert np.array_equal(bits(dc.cpu().numpy()), bits(c)), step
            assert np.array_equal(bits(dd.gp.cpu().numpy()), bits(gp)), step
    finally:
        dd.release()


@pytest.mark.parametrize("model", [False, True])
def test_joint(hip, torch, model):
    dec = decoder(12, model)
    dw = ol.DecoderWeights(dec)
    dd = hip.DeviceDecoder(dec, torch)
    try:
        g = synth.rng(13)
        for i in range(6):
            f, gp = (g.standard_normal((2, dec["J"])) * (1 + i)).astype(np.float32)
            logit, tok, dur = ol.joint(dw, f, gp)
            dd.gp.copy_(dev(torch, gp))
            say("joint", model, i)
            off = i % 2                     # odd steps: f off 16-byte alignment
            dd.joint(dev(torch, np.concatenate([np.zeros(off, np.float32), f]))[off:])
            torch.cuda.synchronize()
            assert np.array_equal(bits(dd.logit.cpu().numpy()), bits(logit)), i
            assert tuple(dd.tok_dur.cpu().numpy().tolist()) == (tok, dur), i
    finally:
        dd.release()


@pytest.mark.parametrize("n_dur", [64, 70])
def test_joint_many_durations(hip, torch, n_dur):
    """Up to 64 durations the argmax scans them from registers (a lane
    each); past 64 from memory: both against the oracle's joint."""
    dec = synth.decoder_weights(synth.rng(17 + n_dur), P=64, L=2, J=64, V=40, n_dur=n_dur)
    dw = ol.DecoderWeights(dec)
    dd = hip.DeviceDecoder(dec, torch)
    try:
        g = synth.rng(19)
        for i in range(4):
            f, gp = (g.standard_normal((2, dec["J"])) * (1 + i)).astype(np.float32)
            logit, tok, dur = ol.joint(dw, f, gp)
            dd.gp.copy_(dev(torch, gp))
            say("joint durations", n_dur, i)
            dd.joint(dev(torch, f))
            torch.cuda.synchronize()
            assert np.array_equal(bits(dd.logit.cpu().numpy()), bits(logit)), i
            assert tuple(dd.tok_dur.cpu().numpy().tolist()) == (tok, dur), i
    finally:
        dd.release()


def test_argmax_rule(hip, torch):
    """Logits placed through the bias of a zero joint matrix: ties go to the
    first, +0 and -0 are equal, a NaN never wins but at index 0, where
    nothing beats it; spread over the lanes' runs (V = 1024)."""
    dec = decoder(14, True)
    V, n_dur = dec["V"], dec["n_dur"]
    dec["jout"] = np.zeros_like(dec["jout"])
    rows = dec["jout_s"].size
    f = np.zeros(dec["J"], np.float32)
    cases = []
    b = np.zeros(rows, np.float32)
    b[17] = b[900] = 3.0
    b[V + 1 + 2] = b[V + 1 + 4] = 1.0
    cases.append(b.copy())
    b = np.zeros(rows, np.float32)
    b[0] = -0.0
    b[600] = 0.0
    cases.append(b.copy())
    b = np.full(rows, -1.0, np.float32)
    b[2] = np.nan
    b[16] = np.nan
    b[17] = 0.5
    b[1000] = 0.5
    cases.append(b.copy())
    b = np.full(rows, -1.0, np.float32)
    b[0] = np.nan
    b[700] = 0.5
    cases.append(b.copy())
    b = np.full(rows, np.nan, np.float32)
    cases.append(b.copy())
    b = (synth.rng(15).standard_normal(rows)).astype(np.float32)
    b[1024] = b[:V + 1].max()
    cases.append(b.copy())
    for k, bias in enumerate(cases):
        dec["jout_b"] = bias
        dw = ol.DecoderWeights(dec)
        _, tok, dur = ol.joint(dw, f, f)
        dd = hip.DeviceDecoder(dec, torch)
        try:
            say("argmax case", k)
            dd.joint(dev(torch, f))
            torch.cuda.synchronize()
            assert tuple(dd.tok_dur.cpu().numpy().tolist()) == (tok, dur), k
        finally:
            dd.release()


def test_greedy_search_on_device(hip, torch):
    """The search over 60 encoder frames with the device's steps and with the
    oracle's: the same tokens, frames and durations."""
    dec = decoder(16, True)
    V, J, L, P = dec["V"], dec["J"], dec["L"], dec["P"]
    durs = [0, 1, 2, 3, 4]
    T = 60
    g = synth.rng(17)
    frames = (g.standard_normal((T, J)) * 2).astype(np.float32)
    blank = V
    dw = ol.DecoderWeights(dec)
    st = {"h": np.zeros((L, P), np.float32), "c": np.zeros((L, P), np.float32), "gp": None}

    def o_predict(k):
        st["h"], st["c"], st["gp"] = ol.predict(dw, k, st["h"], st["c"])

    def o_joint(t):
        _, k, di = ol.joint(dw, frames[t], st["gp"])
        return k, di
    want = search(T, o_predict, o_joint, blank, durs, 10)
    dd = hip.DeviceDecoder(dec, torch)
    try:
        fd = dev(torch, frames)

        def d_joint(t):
            dd.joint(None, f_ptr=fd.data_ptr() + 4 * t * J)
            k, di = dd.tok_dur.cpu().numpy().tolist()
            return k, di
        say("search", T)
        got = search(T, dd.predict, d_joint, blank, durs, 10)
    finally:
        dd.release()
    assert got == want and len(want) > 3


@pytest.mark.parametrize("resident", [True, False])
@pytest.mark.parametrize("T,seed,scale", [(60, 16, 2.0), (300, 21, 1.0), (5, 22, 3.0)])
def test_search_in_one_launch(hip, torch, T, seed, scale, resident):
    """pk_hip_search_dev, the whole search in one cooperative launch, at the
    model's shapes (pred 640, 2 LSTM layers, joint 640, 1024 tokens + blank,
    5 durations): the oracle-driven search's tokens, frames and durations;
    over frames whose scale makes it emit often and others that are mostly
    blank; then the same search again on the same decoder (the state starts
    from zero each call). Both with the panels resident (registers and LDS,
    loaded once a launch) and loaded each token."""
    dec = decoder(seed, True)
    V, J, L, P = dec["V"], dec["J"], dec["L"], dec["P"]
    durs = [0, 1, 2, 3, 4]
    g = synth.rng(seed + 1)
    frames = (g.standard_normal((T, J)) * scale).astype(np.float32)
    blank = V
    dw = ol.DecoderWeights(dec)
    st = {"h": np.zeros((L, P), np.float32), "c": np.zeros((L, P), np.float32), "gp": None}

    def o_predict(k):
        st["h"], st["c"], st["gp"] = ol.predict(dw, k, st["h"], st["c"])

    def o_joint(t):
        _, k, di = ol.joint(dw, frames[t], st["gp"])
        return k, di
    want = search(T, o_predict, o_joint, blank, durs, 10)
    dd = hip.DeviceDecoder(dec, torch)
    was = hip.force_search_resident(resident)
    try:
        fd = dev(torch, frames)
        for call in range(2):
            say("search in one launch", T, seed, call, "resident" if resident else "loaded")
            got = dd.search(fd, T, blank, durs, 10)
            assert got == want, (call, len(got), len(want))
    finally:
        hip.force_search_resident(was)
        dd.release()
    assert len(want) > 0


def test_search_bounded_wait_gives_up(hip, torch):
    """A grid-wide wait whose iteration limit the host sets to 1: the launch
    ends early (every workgroup leaves at its first wait or on the flag), the
    call returns PK_HIP_ETIMEOUT, and the next search on the same device
    with the default limit is whole again."""
    dec = decoder(23, True)
    V, J = dec["V"], dec["J"]
    durs = [0, 1, 2, 3, 4]
    T = 40
    frames = (synth.rng(24).standard_normal((T, J)) * 2).astype(np.float32)
    dd = hip.DeviceDecoder(dec, torch)
    try:
        fd = dev(torch, frames)
        say("search with a wait limit of 1")
        with pytest.raises(hip.PkHipError) as e:
            dd.search(fd, T, V, durs, 10, spin_limit=1)
        assert e.value.code == hip.PK_HIP_ETIMEOUT
        say("search with the default limit")
        again = dd.search(fd, T, V, durs, 10)
        first = dd.search(fd, T, V, durs, 10)
        assert again == first
    finally:
        dd.release()


@pytest.mark.parametrize("P,L,J,V,durs", [(1024, 1, 512, 2000, [0, 1, 2]), (256, 3, 768, 100, [0, 1, 2, 4]),
                                          (320, 2, 320, 500, [0, 1, 2, 3, 4]), (64, 2, 96, 30, [1, 2])])
def test_search_in_one_launch_other_shapes(hip, torch, P, L, J, V, durs):
    """The one-launch search beyond the model's shapes: prediction widths up
    to 1024 (16 units a panel row, where the panels are loaded each token),
    one and three LSTM layers, a joint wider than the prediction, a
    vocabulary of 2000, durations without 0; its tokens, frames and
    durations the oracle-driven search's, with the panels resident where
    they fit and loaded each token everywhere."""
    dec = synth.decoder_weights(synth.rng(P + L + J), P=P, L=L, J=J, V=V, n_dur=len(durs))
    T = 120
    frames = (synth.rng(P + J).standard_normal((T, J)) * 2.0).astype(np.float32)
    blank = V
    dw = ol.DecoderWeights(dec)
    st = {"h": np.zeros((L, P), np.float32), "c": np.zeros((L, P), np.float32), "gp": None}

    def o_predict(k):
        st["h"], st["c"], st["gp"] = ol.predict(dw, k, st["h"], st["c"])

    def o_joint(t):
        _, k, di = ol.joint(dw, frames[t], st["gp"])
        return k, di
    want = search(T, o_predict, o_joint, blank, durs, 10)
    dd = hip.DeviceDecoder(dec, torch)
    try:
        fd = dev(torch, frames)
        for resident in (True, False):
            was = hip.force_search_resident(resident)
            try:
                say("search in one launch", P, L, J, V, len(durs), "resident" if resident else "loaded")
                got = dd.search(fd, T, blank, durs, 10)
            finally:
                hip.force_search_resident(was)
            assert got == want, (resident, len(got), len(want))
    finally:
        dd.release()
    assert len(want) > 0
