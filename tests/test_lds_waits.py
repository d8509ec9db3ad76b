"""The product kernels' LDS reads are inline asm that the compiler takes as
ready at once; the kernels wait for them with explicit lgkmcnt waits. These
CPU tests compile the kernels to gfx950 assembly with the library's own flags
and check that no instruction touches a read's destination before its wait
(tests/lds_waits.py), on every path of every kernel that issues such reads."""
import os
import subprocess

import pytest

import lds_waits

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_analysis_catches_a_copy_before_the_wait():
    body = """
        ds_read_b128 v[4:7], v1
        ds_read_b128 v[8:11], v2
        s_waitcnt lgkmcnt(1)
        v_mov_b32_e32 v20, v4
        v_mov_b32_e32 v21, v9
        s_waitcnt lgkmcnt(0)
        v_mov_b32_e32 v22, v9
        s_endpgm
    """.split("\n")
    bad = lds_waits.violations(body)
    assert [t for t, _ in bad] == ["v_mov_b32_e32 v21, v9"]


def test_analysis_follows_loops_and_joins():
    # the read issued at the bottom of the loop is in flight at its top
    body = """
        s_waitcnt lgkmcnt(0)
    .LBB0_1:
        v_add_u32_e32 v30, v12, v13
        ds_read_b128 v[12:15], v3
        s_cbranch_scc1 .LBB0_1
        s_waitcnt lgkmcnt(0)
        v_mov_b32_e32 v1, v12
        s_endpgm
    """.split("\n")
    bad = lds_waits.violations(body)
    assert [t for t, _ in bad] == ["v_add_u32_e32 v30, v12, v13"]
    ok = [l.replace("v_add_u32_e32 v30, v12, v13", "s_waitcnt lgkmcnt(0)") for l in body]
    assert lds_waits.violations(ok) == []


def _asm(tmp_path_factory, src):
    from libpktito_amd import build
    out = tmp_path_factory.mktemp("asm") / (os.path.basename(src) + ".s")
    cmd = [build.HIPCC] + build.flags_for(src) + ["--cuda-device-only", "-S", src, "-o", str(out),
                                                  "-I", os.path.join(ROOT, "include"),
                                                  "-I", os.path.dirname(src)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out.read_text()


@pytest.fixture(scope="module")
def kernels_asm(tmp_path_factory):
    from libpktito_amd import build
    return _asm(tmp_path_factory, next(s for s in build.SOURCES if s.endswith("q8_kernels.hip")))


def test_product_kernels_wait_before_touching_lds_reads(kernels_asm):
    fns = lds_waits.functions(kernels_asm, r"gemm_(ring|pipe)_(grouped_)?kernel")
    assert any("ring" in n for n in fns) and any("pipe" in n for n in fns), sorted(fns)
    bad = {name: v[:2] for name, v in ((n, lds_waits.violations(b)) for n, b in fns.items()) if v}
    assert not bad, bad


@pytest.fixture(scope="module")
def stream_asm(tmp_path_factory):
    from libpktito_amd import build
    return _asm(tmp_path_factory, next(s for s in build.SOURCES if s.endswith("q8_stream.hip")))


def test_streamed_kernels_wait_before_touching_lds_reads(stream_asm):
    fns = lds_waits.functions(stream_asm, r"gemm_stream_kernel")
    assert fns, "no streamed kernel in the assembly"
    bad = {name: v[:2] for name, v in ((n, lds_waits.violations(b)) for n, b in fns.items()) if v}
    assert not bad, bad


def test_streamed_kernels_mfma_loop_never_waits_on_vmcnt(stream_asm):
    """The streamed kernels' MFMA waves issue no global loads in their K loop,
    and their stores drain under the next tile's loop only if nothing there
    waits on vmcnt (which counts stores too): no basic block that holds an
    MFMA may hold a vmcnt wait (a residual load left in flight across a tile,
    or a spill, would put one there)."""
    fns = lds_waits.functions(stream_asm, r"gemm_stream_kernel")
    for name, body in fns.items():
        blocks, _ = lds_waits._blocks(body)
        mfma = [b for b in blocks if any(t.startswith("v_mfma") for t in b)]
        assert mfma, name
        waits = [t for b in mfma for t in b if t.startswith("s_waitcnt") and "vmcnt" in t]
        assert not waits, (name, waits[:3])
        assert "scratch_" not in "\n".join(body), name
