"""backend/hip's table inside the reference's own library, on the GPU.

oracle/Makefile compiles the reference's library (its Makefile's LIB_SRC,
where the files lie, unedited) with the table libpktito_amd/backend_hip/
kernels.c and its upload step (model_upload.c) into three programs under
oracle/_ref: the reference's own parity checkers tests/kcheck.c and
tests/q8check.c, which test every table of the registry whose needs the
machine meets against ref (the hip table among them when a GPU opens), and
dropin_cli, a transcription (core/asr.c's pk_asr_run: the encoder of
core/encoder.c and the decoder) on whichever table PKTITO_KERNELS names,
printed token by token. The model is tests/golden/tiny.pkf, the
reference's tests/data/tiny.pkf (d_model 64, two layers: every product of
the encoder and the decoder goes through the table); for the diarizer,
tests/golden/tiny-diar.pkf, the reference's tests/data/tiny-diar.pkf.

Bit for bit, as the reference holds every backend (backend/kernels.h:9-14):
kcheck's and q8check's verdict lines, and the transcripts compared with cmp's
strictness as tests/check-c.sh:73-81 does."""
import os
import re
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref")
TINY = os.path.join(ROOT, "tests", "golden", "tiny.pkf")
HIP_NAME = "hip (MI355X gfx950"


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def program(name):
    p = os.path.join(REF, name)
    if not os.path.exists(p):
        pytest.skip(f"{p} was not built (the reference checkout was absent when build() ran)")
    return p


def sections(out):
    """{table name: (cases, verdict, FAIL lines before its summary line)}"""
    res, pending = {}, []
    for line in out.splitlines():
        m = re.match(r"(kcheck|q8check): (.*), (\d+) cases(?: at guard pages)?: (.*)$", line)
        if m:
            res[m.group(2)] = (int(m.group(3)), m.group(4), pending)
            pending = []
        elif line.startswith("FAIL"):
            pending.append(line)
    return res


def hip_section(sec):
    names = [n for n in sec if n.startswith(HIP_NAME)]
    assert names, f"the hip table was not tested: {sorted(sec)}"
    return sec[names[0]]


def test_q8check_holds_the_hip_table_to_ref():
    """tests/q8check.c: 385 cases of gemm_q8 with every operand against
    PROT_NONE guard pages (no byte read or written past them), bias, add,
    output pitches, a run of panels, T = 0 and the three directed roundings:
    the hip table's outputs are ref's, every one."""
    say("q8check")
    r = subprocess.run([program("q8check")], capture_output=True, text=True, timeout=600)
    sec = sections(r.stdout)
    cases, verdict, fails = hip_section(sec)
    assert verdict == "every one ref's bits" and not fails, r.stdout[-3000:]
    assert cases >= 385
    assert r.returncode == 0, r.stdout[-3000:]


def test_kcheck_holds_the_hip_table_to_ref():
    """tests/kcheck.c without a model: the quantizer's cases (non-finite
    blocks, the 2^-121 edge, xs > n, blocks of 32 and 64 and whole columns)
    and gemm_q8's (random shapes, qb, bias, add, pitches, interior panels,
    the x86 backends' tile edges), each a buffer of kcheck's own (the
    table copies and repacks weights it was not given at upload), plus the
    float kernels the table takes from the CPU."""
    say("kcheck")
    r = subprocess.run([program("kcheck")], capture_output=True, text=True, timeout=900)
    cases, verdict, fails = hip_section(sections(r.stdout))
    assert verdict == "every one ref's bits" and not fails, r.stdout[-3000:]
    assert cases >= 1738
    assert r.returncode == 0, r.stdout[-3000:]


def test_kcheck_model_cases_on_tiny_pkf():
    """kcheck with the model (tests/kcheck.c:475-494): the middle layer's
    ff1_up, ff1_down, q, o, pw1, jout and the first LSTM's wx, as the
    loaded model binds them, in blocks of 32 and of 64. The run draws its
    later cases from where the model's leave the generator, and one of
    those (quant_tiny_case, :150-176) then writes a zero over the block's
    largest value: its check of ref's own scale fails for every table
    alike. So the hip table's section must be every CPU table's: the same
    cases and the same failure lines, and no comparison with ref failing."""
    say("kcheck tiny.pkf")
    r = subprocess.run([program("kcheck"), TINY], capture_output=True, text=True, timeout=900)
    sec = sections(r.stdout)
    hcases, hverdict, hfails = hip_section(sec)
    cpu = {n: v for n, v in sec.items() if not n.startswith(HIP_NAME)}
    assert cpu, r.stdout[-3000:]
    for name, (cases, verdict, fails) in cpu.items():
        assert hcases == cases and hfails == fails, (name, hcases, cases, hfails, fails)
    assert all(f.startswith("FAIL tiny quantize: block of 0x1p-121") for f in hfails), hfails


@pytest.mark.parametrize("whole", [0, 1])
@pytest.mark.parametrize("seconds,seed,fast", [(20, 1, 0), (20, 2, 1), (7, 3, 0)])
def test_transcript_on_the_hip_table_is_refs(seconds, seed, fast, whole):
    """A transcription through the reference's unedited encoder and decoder
    (core/asr.c pk_asr_run, core/encoder.c, core/decoder.c) on 8 threads,
    whose pool deals the products to the table from every thread at once:
    the tokens and their frames and durations, byte for byte, are those of
    the run on ref; with the model uploaded at load and released before it
    is freed. In blocks of 32 and, fast, of 64. whole 1: the harness built
    with the core/passes.c change (oracle/whole_product.c), which hands the
    table each product and each quantize whole."""
    cli = program("dropin_cli_whole" if whole else "dropin_cli")
    outs = {}
    for table in ("ref", "hip"):
        say("transcript", table, seconds, seed, fast)
        env = dict(os.environ, PKTITO_KERNELS=table)
        r = subprocess.run([cli, TINY, str(seconds), str(seed), str(fast), "8"], capture_output=True, text=True,
                           env=env, timeout=600)
        assert r.returncode == 0, (table, r.stderr[-2000:])
        assert table in r.stderr.split("backend:")[-1], r.stderr
        outs[table] = r.stdout
    assert outs["hip"].startswith("tokens ") and int(outs["hip"].split()[1]) > 0
    assert outs["hip"] == outs["ref"]


TINY_DIAR = os.path.join(ROOT, "tests", "golden", "tiny-diar.pkf")


@pytest.mark.parametrize("whole", [0, 1])
@pytest.mark.parametrize("seconds,seed", [(20, 1), (40, 2)])
def test_diarization_on_the_hip_table_is_refs(seconds, seed, whole):
    """The reference's second caller of the table: its diarizer (core/diar.c,
    pk_diar_run: the transformer layers' q, k, v, o and feed-forward
    products, the projection, the upsampling and the head, every one
    pk_k_gemm_q8 on activations quantized in blocks of 32) on
    tests/golden/tiny-diar.pkf, the reference's tests/data/tiny-diar.pkf,
    on 8 threads. Every row of speaker probabilities, as exact hex floats,
    is the run on ref's; with the diarizer's matrices uploaded at load (the
    walker's diarizer branch) and released before the free. 40 s cross the
    model's 27.2 s chunk, so the speaker cache carries between chunks.
    whole 1: with the core/passes.c change, as above."""
    cli = program("dropin_cli_whole" if whole else "dropin_cli")
    outs = {}
    for table in ("ref", "hip"):
        say("diarization", table, seconds, seed)
        env = dict(os.environ, PKTITO_KERNELS=table)
        r = subprocess.run([cli, TINY_DIAR, str(seconds), str(seed), "0", "8"], capture_output=True, text=True,
                           env=env, timeout=600)
        assert r.returncode == 0, (table, r.stderr[-2000:])
        assert table in r.stderr.split("backend:")[-1], r.stderr
        outs[table] = r.stdout
    last = outs["hip"].strip().splitlines()[-1].split()
    assert last[0] == "rows" and int(last[1]) >= seconds * 25 and int(last[2]) > 0, last
    assert outs["hip"] == outs["ref"]


def test_whole_product_passes_time_through_the_pool():
    """The reference's own pool entries (pk_quantize_on, pk_gemm_on) on a
    synthetic 750 x 1024 -> 4096 product, through both harnesses on the hip
    table and on ref's neighbour avx512-vnni: every run ends, the same
    outputs (a checksum) on every table and dealing, and the whole-product
    harness makes one call a product under hip (a handful of milliseconds at
    most; the timings themselves are the bench's)."""
    import json
    res = {}
    for whole in (0, 1):
        cli = program("dropin_cli_whole" if whole else "dropin_cli")
        for table in ("hip", "avx512-vnni"):
            say("time passes", whole, table)
            env = dict(os.environ, PKTITO_KERNELS=table)
            r = subprocess.run([cli, "--time-passes", "8", "0.3"], capture_output=True, text=True, env=env,
                               timeout=300)
            if table != "hip" and r.returncode != 0 and "does not have" in r.stderr:
                continue
            assert r.returncode == 0, (whole, table, r.stderr[-2000:])
            res[(whole, table)] = json.loads(r.stdout.strip().splitlines()[-1])
    checks = {v["check"] for v in res.values()}
    assert len(checks) == 1, res
    assert res[(1, "hip")]["pair_ms"] < 5.0, res
