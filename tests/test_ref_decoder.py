"""The oracle's decoder against the reference's own.

oracle/dropin_cli.c runs a transcription of tests/golden/tiny.pkf through
the reference's library (built in place by oracle/Makefile) on its ref
table, and writes the decoder's input (the joint's encoder half of every
frame, core/decoder.c:149-156), the prediction network and joint weights,
and the tokens the reference's search emitted (core/decoder.c:121-147).
The same greedy search driven by the oracle's prediction and joint steps
(pko_predict_with, pko_joint_with: core/decoder.c:67-101) over the same
frames must emit the same tokens, frames and durations. This pins the
oracle's decoder steps, which the device's steps are held to, to the
reference's decoder itself. CPU only."""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as ol
from tdt_search import search

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "oracle", "_ref", "dropin_cli")
TINY = os.path.join(ROOT, "tests", "golden", "tiny.pkf")


def read_dump(path):
    raw = open(path, "rb").read()
    assert raw[:4] == b"PKDC"
    off = 4

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(raw, dtype=dtype, count=count, offset=off).copy()
        off += a.nbytes
        return a

    def q8(dec, name):
        rows, cols = (int(v) for v in take(np.uint32, 2))
        dec[name] = take(np.int8, rows * cols)
        dec[name + "_s"] = take(np.float32, rows)
        return rows

    Te, P, L, J, V, n_dur, blank, max_symbols = (int(v) for v in take(np.uint32, 8))
    durs = [int(v) for v in take(np.uint32, n_dur)]
    f = take(np.float32, Te * J).reshape(Te, J)
    dec = dict(P=P, L=L, J=J, V=V, n_dur=n_dur)
    dec["embed"] = take(np.float32, (V + 1) * P)
    for l in range(L):
        q8(dec, f"wx{l}")
        q8(dec, f"wh{l}")
        dec[f"b{l}"] = take(np.float32, 4 * P)
    q8(dec, "jpred")
    dec["jpred_b"] = take(np.float32, J)
    rows = q8(dec, "jout")
    dec["jout_b"] = take(np.float32, rows)
    jenc = {}
    q8(jenc, "jenc")
    jenc["jenc_b"] = take(np.float32, J)
    n = int(take(np.uint32, 1)[0])
    toks = [tuple(int(v) for v in take(np.int32, 3)) for _ in range(n)]
    assert off == len(raw)
    return dict(Te=Te, f=f, dec=dec, jenc=jenc, blank=blank, durs=durs, max_symbols=max_symbols, toks=toks)


def reference_decoder(tmp_path, seconds, seed, fast):
    """(the dump, the harness's stdout) of a transcription on ref"""
    if not os.path.exists(CLI):
        pytest.skip("oracle/_ref/dropin_cli was not built (the reference checkout was absent when build() ran)")
    out = tmp_path / "decoder.bin"
    env = dict(os.environ, PKTITO_KERNELS="ref")
    r = subprocess.run([CLI, TINY, str(seconds), str(seed), str(fast), "8", "--decoder", str(out)],
                       capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    return read_dump(out), r.stdout


@pytest.mark.parametrize("seconds,seed,fast", [(7, 3, 0), (20, 1, 0), (20, 2, 1)])
def test_oracle_decoder_is_the_references(tmp_path, seconds, seed, fast):
    d, stdout = reference_decoder(tmp_path, seconds, seed, fast)
    dec = d["dec"]
    dw = ol.DecoderWeights(dec)
    st = {"h": np.zeros((dec["L"], dec["P"]), np.float32), "c": np.zeros((dec["L"], dec["P"]), np.float32),
          "gp": None}

    def predict(k):
        st["h"], st["c"], st["gp"] = ol.predict(dw, k, st["h"], st["c"])

    def joint(t):
        _, k, di = ol.joint(dw, d["f"][t], st["gp"])
        return k, di
    got = search(d["Te"], predict, joint, d["blank"], d["durs"], d["max_symbols"])
    assert len(d["toks"]) > 5
    assert got == d["toks"]
    # and the transcript the harness printed is the same search's
    printed = [tuple(int(v) for v in line.split()) for line in stdout.splitlines()[1:]]
    assert printed == d["toks"]


@pytest.mark.gpu
@pytest.mark.parametrize("seconds,seed,fast", [(7, 3, 0), (20, 2, 1)])
def test_device_decoder_is_the_references(hip, tmp_path, seconds, seed, fast):
    """The device's token steps (pk_hip_lstm_step_dev, pk_hip_joint_dev and
    the jpred gemv, in DeviceDecoder) driving the same search over the
    reference's joint frames of tiny.pkf: the reference's tokens."""
    import torch
    d, _ = reference_decoder(tmp_path, seconds, seed, fast)
    dd = hip.DeviceDecoder(d["dec"], torch)
    try:
        fd = torch.from_numpy(np.ascontiguousarray(d["f"])).cuda()
        J = d["dec"]["J"]

        def joint(t):
            dd.joint(None, f_ptr=fd.data_ptr() + 4 * t * J)
            k, di = dd.tok_dur.cpu().numpy().tolist()
            return k, di
        print("[case] device search", seconds, seed, fast, flush=True)
        got = search(d["Te"], dd.predict, joint, d["blank"], d["durs"], d["max_symbols"])
    finally:
        dd.release()
    assert got == d["toks"] and len(got) > 5


@pytest.mark.gpu
@pytest.mark.parametrize("seconds,seed,fast", [(7, 3, 0), (20, 1, 0), (20, 2, 1)])
def test_device_search_is_the_references(hip, tmp_path, seconds, seed, fast):
    """The whole search in one launch on the device (pk_hip_search_dev:
    the LSTM layers, jpred, the joint, its argmax and the duration step
    with no host round trip) over the reference's joint frames of tiny.pkf:
    the reference's tokens, frames and durations."""
    import torch
    d, _ = reference_decoder(tmp_path, seconds, seed, fast)
    dd = hip.DeviceDecoder(d["dec"], torch)
    try:
        fd = torch.from_numpy(np.ascontiguousarray(d["f"])).cuda()
        print("[case] device search in one launch", seconds, seed, fast, flush=True)
        got = dd.search(fd, d["Te"], d["blank"], d["durs"], d["max_symbols"])
    finally:
        dd.release()
    assert got == d["toks"] and len(got) > 5
