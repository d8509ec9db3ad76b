"""The drop-in harness without a GPU (test_gpu_dropin.py runs it on one):
the reference's library built in place with backend/hip's table
(oracle/Makefile, _ref/dropin_cli, _ref/kcheck, _ref/q8check) gives the same
transcript, and the same diarization, on two of its CPU tables, and where no device opens the hip
table is refused, as its needs say, and skipped by the reference's checkers,
never run on the CPU instead."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.path.join(ROOT, "oracle", "_ref")
TINY = os.path.join(ROOT, "tests", "golden", "tiny.pkf")
NODEV = dict(os.environ, PKTITO_HIP_DISABLE="1")


def program(name):
    p = os.path.join(REF, name)
    if not os.path.exists(p):
        pytest.skip(f"{p} was not built (no reference checkout when oracle/ was built)")
    return p


def transcript(table, *args):
    r = subprocess.run([program("dropin_cli"), TINY, *args], capture_output=True, text=True,
                       env=dict(NODEV, PKTITO_KERNELS=table), timeout=300)
    return r


def test_cpu_tables_give_one_transcript():
    a = transcript("ref", "12", "4", "0", "4")
    b = transcript("avx2", "12", "4", "0", "4")
    assert a.returncode == 0 and b.returncode == 0, (a.stderr, b.stderr)
    assert a.stdout.startswith("tokens ") and a.stdout == b.stdout


def test_hip_table_is_refused_without_a_device():
    r = transcript("hip", "1", "1", "0", "1")
    assert r.returncode != 0
    assert "PKTITO_KERNELS=hip uses hip, which this CPU does not have" in r.stderr


def test_checkers_skip_the_hip_table_without_a_device():
    r = subprocess.run([program("q8check")], capture_output=True, text=True, env=NODEV, timeout=600)
    assert "hip (MI355X gfx950" in r.stdout and "this CPU has no hip - skipped" in r.stdout, r.stdout
    assert r.returncode == 0, r.stdout[-2000:]


def test_cpu_tables_give_one_diarization():
    """The harness's diarizer run (tests/golden/tiny-diar.pkf, the
    reference's tests/data/tiny-diar.pkf): every row of speaker
    probabilities, as hex floats, alike on two CPU tables."""
    diar = os.path.join(ROOT, "tests", "golden", "tiny-diar.pkf")
    runs = [subprocess.run([program("dropin_cli"), diar, "8", "5", "0", "4"], capture_output=True, text=True,
                           env=dict(NODEV, PKTITO_KERNELS=t), timeout=300) for t in ("ref", "avx2")]
    assert all(r.returncode == 0 for r in runs), [r.stderr for r in runs]
    last = runs[0].stdout.strip().splitlines()[-1].split()
    assert last[0] == "rows" and int(last[1]) > 0 and runs[0].stdout.count("row ") == int(last[1])
    assert runs[0].stdout == runs[1].stdout
