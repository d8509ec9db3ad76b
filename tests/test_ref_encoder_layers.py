"""The oracle's and the device's encoder layer against the reference's own.

oracle/Makefile builds the reference's library where its files lie, with
the harness oracle/dropin_cli.c, which runs the reference's encoder
(core/encoder.c: pk_encode, :429-506, whose layer function, :338-368, is
static) on tests/golden/tiny.pkf with the model's n_layers set to 0, 1 and
2 in turn on the same features, through the reference's ref table
(PKTITO_KERNELS=ref), and writes each layer's input and output, the
positions' quantized encodings and the layers' weights. The oracle's
pko_conformer_layer, given the same input, encodings and weights, must give
the reference's output bits, for both layers and in both of the encoder's
block sizes (32, and 64 in its fast mode). This pins the oracle's
composition of the layer (the order of its passes, which activation each
product reads, where the residuals add) to the reference's encoder itself,
not to a second restatement; and the device-resident layer
(pk_hip_layer_dev) to the same outputs, on the GPU."""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as ol

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "oracle", "_ref", "dropin_cli")
TINY = os.path.join(ROOT, "tests", "golden", "tiny.pkf")


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def read_dump(path):
    raw = open(path, "rb").read()
    assert raw[:4] == b"PKLD"
    off = 4

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(raw, dtype=dtype, count=count, offset=off).copy()
        off += a.nbytes
        return a

    Te, D, H, F, K, qb, L = (int(v) for v in take(np.uint32, 7))
    eps = float(take(np.float32, 1)[0])
    xs = [take(np.float32, Te * D).reshape(Te, D) for _ in range(L + 1)]
    R = 2 * Te - 1
    ape_q = take(np.int8, R * D)
    ape_d = take(np.float32, R * (D // qb))
    pe = take(np.float32, R * D).reshape(R, D)
    layers = []
    for _ in range(L):
        w = dict(D=D, H=H, F=F, K=K, eps=eps)
        for n in ol.LAYER_NORMS + ("bias_u", "bias_v"):
            w[n] = take(np.float32, D)
        w["dw"] = take(np.float32, D * K)
        w["dw_b"] = take(np.float32, D)
        for n in ol.LAYER_MATS:
            rows, cols = (int(v) for v in take(np.uint32, 2))
            w[n] = take(np.int8, rows * cols)
            w[n + "_s"] = take(np.float32, rows)
        layers.append(w)
    assert off == len(raw)
    return dict(Te=Te, qb=qb, xs=xs, ape_q=ape_q, ape_d=ape_d, pe=pe, layers=layers)


def reference_layers(tmp_path, fast):
    if not os.path.exists(CLI):
        pytest.skip("oracle/_ref/dropin_cli was not built (the reference checkout was absent when build() ran)")
    out = tmp_path / "layers.bin"
    env = dict(os.environ, PKTITO_KERNELS="ref")
    r = subprocess.run([CLI, TINY, "7", "3", str(fast), "8", "--layers", str(out)], capture_output=True, text=True,
                       env=env, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "ref" in r.stderr.split("backend:")[-1]
    return read_dump(out)


@pytest.mark.parametrize("fast", [0, 1])
def test_oracle_layer_is_the_reference_encoders(tmp_path, fast):
    dump = reference_layers(tmp_path, fast)
    assert dump["qb"] == (64 if fast else 32) and len(dump["layers"]) == 2
    Te = dump["Te"]
    for i, w in enumerate(dump["layers"]):
        x_in, want = dump["xs"][i], dump["xs"][i + 1]
        assert np.isfinite(want).all() and not np.array_equal(bits(x_in), bits(want))
        got = ol.conformer_layer(w, x_in, Te, dump["ape_q"], dump["ape_d"], dump["qb"], threads=4)
        assert np.array_equal(bits(got), bits(want)), (fast, i)


@pytest.mark.gpu
@pytest.mark.parametrize("valu", [0, 1])
@pytest.mark.parametrize("fast", [0, 1])
def test_device_layer_is_the_reference_encoders(hip, tmp_path, fast, valu):
    """pk_hip_layer_dev (the whole layer in HBM) on the same input, the
    reference's positional encodings quantized on the device (which must
    give the reference's bytes and scales) and the same weights: the
    reference's output bits, for both layers. The tiny model's heads are 16
    wide, so the attention runs on its one-thread-an-output kernels (whose
    output is quantized by a pass of its own) whatever valu sets."""
    import torch
    dump = reference_layers(tmp_path, fast)
    Te, qb = dump["Te"], dump["qb"]
    D = dump["layers"][0]["D"]
    R = 2 * Te - 1
    ape_q = torch.empty((R, D), dtype=torch.int8, device="cuda")
    ape_qp = torch.zeros((hip.packed_bytes(D, R),), dtype=torch.int8, device="cuda")
    ape_d = torch.empty((R * (D // qb),), dtype=torch.float32, device="cuda")
    hip.quantize_packed_dev(ape_q, ape_qp, ape_d, torch.from_numpy(dump["pe"]).cuda(), D, R, D, qb=qb)
    torch.cuda.synchronize()
    assert np.array_equal(ape_q.cpu().numpy().reshape(-1), dump["ape_q"])
    assert np.array_equal(bits(ape_d.cpu().numpy()), bits(dump["ape_d"]))
    was = hip.force_attention(valu)
    try:
        for i, w in enumerate(dump["layers"]):
            lay = hip.DeviceLayer(w, torch)
            try:
                ws = torch.empty((lay.workspace(Te, qb),), dtype=torch.uint8, device="cuda")
                xt = torch.from_numpy(np.ascontiguousarray(dump["xs"][i])).cuda()
                print("[case] device layer", fast, valu, i, flush=True)
                lay.run(xt, Te, ape_qp, ape_d, qb, ws)
                torch.cuda.synchronize()
                got = xt.cpu().numpy()
            finally:
                lay.release()
            assert np.array_equal(bits(got), bits(dump["xs"][i + 1])), (fast, valu, i)
    finally:
        hip.force_attention(was)
