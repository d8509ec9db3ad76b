"""A transcription's device-resident path against the reference's own.

For the same recording of tests/golden/tiny.pkf the harness
(oracle/dropin_cli.c, the reference's library built in place, on its ref
table) writes the encoder's input after the subsampling, each layer's
output and the weights (test_ref_encoder_layers.py), and the joint's
encoder half of every frame, the decoder's weights and the emitted tokens
(test_ref_decoder.py). On the device: both encoder layers
(pk_hip_layer_dev), the per-row quantize and the joint's encoder product
of pk_joint_frames (core/decoder.c:149-156: quantize with qb = d_model,
gemm_q8 with jenc and its bias), then the greedy search over the device's
prediction and joint steps. Every stage gives the reference's bits, and
the tokens, frames and durations are the reference's transcript."""
import numpy as np
import pytest

from tdt_search import search
from test_ref_decoder import reference_decoder
from test_ref_encoder_layers import bits, reference_layers

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fast", [0, 1])
def test_device_path_transcribes_as_the_reference(hip, tmp_path, fast):
    import torch
    lay_dump = reference_layers(tmp_path, fast)
    dec_dump, _ = reference_decoder(tmp_path, 7, 3, fast)
    Te, qb = lay_dump["Te"], lay_dump["qb"]
    D = lay_dump["layers"][0]["D"]
    J = dec_dump["dec"]["J"]
    assert dec_dump["Te"] == Te
    R = 2 * Te - 1
    print("[case] device transcript", fast, flush=True)
    ape_qp = torch.zeros((hip.packed_bytes(D, R),), dtype=torch.int8, device="cuda")
    ape_d = torch.empty((R * (D // qb),), dtype=torch.float32, device="cuda")
    hip.quantize_packed_dev(None, ape_qp, ape_d, torch.from_numpy(lay_dump["pe"]).cuda(), D, R, D, qb=qb)
    x = torch.from_numpy(np.ascontiguousarray(lay_dump["xs"][0])).cuda()
    for w in lay_dump["layers"]:
        lay = hip.DeviceLayer(w, torch)
        try:
            ws = torch.empty((lay.workspace(Te, qb),), dtype=torch.uint8, device="cuda")
            lay.run(x, Te, ape_qp, ape_d, qb, ws)
            torch.cuda.synchronize()
        finally:
            lay.release()
    assert np.array_equal(bits(x.cpu().numpy()), bits(lay_dump["xs"][-1]))
    # pk_joint_frames: the encoder's output quantized per row, times jenc
    jenc = dec_dump["jenc"]
    q = torch.empty((Te, D), dtype=torch.int8, device="cuda")
    d = torch.empty((Te,), dtype=torch.float32, device="cuda")
    f = torch.empty((Te, J), dtype=torch.float32, device="cuda")
    jb = torch.from_numpy(jenc["jenc_b"]).cuda()
    hip.quantize_dev(q, d, x, D, D, Te, D)
    with hip.Q8Matrix(jenc["jenc"], jenc["jenc_s"]) as m:
        hip.gemm_q8_dev(f, J, m, 0, J, None, jb, q, d, D, D, Te, 0, ws_ptr=m.dev_scales)
        torch.cuda.synchronize()
    assert np.array_equal(bits(f.cpu().numpy()), bits(dec_dump["f"]))
    dd = hip.DeviceDecoder(dec_dump["dec"], torch)
    try:
        def joint(t):
            dd.joint(None, f_ptr=f.data_ptr() + 4 * t * J)
            k, di = dd.tok_dur.cpu().numpy().tolist()
            return k, di
        got = search(Te, dd.predict, joint, dec_dump["blank"], dec_dump["durs"], dec_dump["max_symbols"])
    finally:
        dd.release()
    assert got == dec_dump["toks"] and len(got) > 5
