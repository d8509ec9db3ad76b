"""pk_hip_attention_noalloc_dev, the attention with its scores in the
library's static scratch, against pk_hip_attention_dev with a workspace of
its own, bit for bit: two calls in a row on the same GPU, the second on
fewer frames (the scratch then still holds the first call's scores past the
second's rows, which no kernel may read), on the matrix-core kernels and the
VALU chains; and the sizes past the scratch refused before anything runs."""
import sys

import numpy as np
import pytest

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


def operands(torch, T, D, seed):
    g = synth.rng(seed)
    q, k, v = (g.standard_normal((3, T, D)) * 1.5).astype(np.float32)
    p = g.standard_normal((2 * T - 1, D)).astype(np.float32)
    bu, bv = (0.3 * g.standard_normal((2, D))).astype(np.float32)
    return [torch.from_numpy(a).cuda() for a in (q, k, v, p, bu, bv)]


@pytest.mark.parametrize("valu", [0, 1])
def test_noalloc_attention_is_the_workspace_ones(hip, torch, valu):
    was = hip.force_attention(valu)
    try:
        for T, D, H in ((750, 1024, 8), (37, 128, 2)):
            ops = operands(torch, T, D, 31 * T + valu)
            ws = torch.empty((hip.attention_workspace(T, H),), dtype=torch.uint8, device="cuda")
            want = torch.full((T, D), 9.0, dtype=torch.float32, device="cuda")
            got = torch.full((T, D), 7.0, dtype=torch.float32, device="cuda")
            say("attention with a workspace", T, D, H, valu)
            hip.attention_dev(want, *ops, T, D, H, ws)
            say("attention in the static scratch", T, D, H, valu)
            hip.attention_noalloc_dev(got, *ops, T, D, H)
            torch.cuda.synchronize()
            w = want.cpu().numpy()
            assert np.isfinite(w).all() and np.count_nonzero(w) > 0.99 * w.size
            assert np.array_equal(bits(got.cpu().numpy()), bits(w)), (T, D, H, valu)
    finally:
        hip.force_attention(was)


def test_noalloc_attention_refuses_sizes_past_the_scratch(hip, torch):
    """884 frames of 8 heads fit the 24 MiB, 885 do not (checked on the
    host: nothing is launched)."""
    lim = 24 << 20
    assert hip.attention_workspace(884, 8) <= lim < hip.attention_workspace(885, 8)
    D, H = 512, 8
    t = torch.zeros((2 * 885, D), dtype=torch.float32, device="cuda")
    with pytest.raises(hip.PkHipError):
        hip.attention_noalloc_dev(t, t, t, t, t, t, t, 885, D, H)
    with pytest.raises(hip.PkHipError):
        hip.attention_noalloc_dev(t, t, t, t, t, t, t, 64, 80, 2)        # heads of 40 dimensions
    hip.attention_noalloc_dev(t, t, t, t, t, t, t, 0, D, H)              # no frames: nothing to do
    torch.cuda.synchronize()


def test_noalloc_attention_under_graph_capture(hip, torch):
    """The entry captured into a HIP graph (what it exists for), replayed
    several times with eager work of the library between replays and new
    inputs copied in before each: every replay's output is
    pk_hip_attention_dev's on the same inputs, bit for bit."""
    T, D, H = 300, 512, 8
    ops = operands(torch, T, D, 77)
    ws = torch.empty((hip.attention_workspace(T, H),), dtype=torch.uint8, device="cuda")
    got = torch.zeros((T, D), dtype=torch.float32, device="cuda")
    say("attention captured", T, D, H)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        hip.attention_noalloc_dev(got, *ops, T, D, H)     # once outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        hip.attention_noalloc_dev(got, *ops, T, D, H)
    torch.cuda.synchronize()
    for rep in range(4):
        fresh = operands(torch, T, D, 1000 + rep)
        for dst, src in zip(ops, fresh):
            dst.copy_(src)
        want = torch.full((T, D), 5.0, dtype=torch.float32, device="cuda")
        say("eager attention between replays", rep)
        hip.attention_dev(want, *ops, T, D, H, ws)
        # an eager call of the entry itself on other frames, so the scratch
        # holds other scores when the replay starts
        other = operands(torch, 64, D, 2000 + rep)
        junk = torch.empty((64, D), dtype=torch.float32, device="cuda")
        hip.attention_noalloc_dev(junk, *other, 64, D, H)
        torch.cuda.synchronize()
        got.fill_(7.0)
        torch.cuda.synchronize()
        say("replay", rep)
        g.replay()
        torch.cuda.synchronize()
        w = want.cpu().numpy()
        assert np.isfinite(w).all()
        assert np.array_equal(bits(got.cpu().numpy()), bits(w)), rep
