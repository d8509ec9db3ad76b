"""The C ABI without a GPU: libpkhip.so builds and loads, exports every function
include/pk_hip.h declares, the Python binding covers them, and the no-device
path fails loudly rather than falling back."""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pk_hip.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(pk_hip_\w+)\s*\(", src)))


@pytest.fixture(scope="module")
def so():
    import libpktito_amd
    if not os.path.exists(libpktito_amd.LIB_PATH):
        from libpktito_amd import build
        build.build()
    return libpktito_amd.LIB_PATH


def test_header_declares_the_path():
    names = declared()
    for must in ("pk_hip_quantize", "pk_hip_gemm_q8", "pk_hip_upload_q8", "pk_hip_release_q8",
                 "pk_hip_quantize_dev", "pk_hip_gemm_q8_dev", "pk_hip_gemm_q8_grouped_dev"):
        assert must in names


def test_every_declared_symbol_is_exported(so):
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (pk_hip_\w+)", out))
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing


def test_python_binding_covers_the_header(so):
    import libpktito_amd
    assert sorted(libpktito_amd._SIGS) == declared()
    libpktito_amd.lib()     # loads, and every signature resolves


def test_no_device_fails_loudly(so):
    """PKTITO_HIP_DISABLE stands in for a host without the GPU: every entry
    returns PK_HIP_ENODEV and the Python side raises; nothing computes on the
    CPU instead."""
    code = (
        "import numpy as np, libpktito_amd as pk\n"
        "try:\n"
        "    pk.init()\n"
        "except pk.PkHipError as e:\n"
        "    assert e.code == pk.PK_HIP_ENODEV, e\n"
        "else:\n"
        "    raise SystemExit('init succeeded')\n"
        "q = np.zeros(32, np.int8); d = np.zeros(1, np.float32)\n"
        "a = pk.make_act(q, d, 32, 32, 1)\n"
        "try:\n"
        "    pk.quantize(a, np.ones(32, np.float32), 32)\n"
        "except pk.PkHipError as e:\n"
        "    assert e.code == pk.PK_HIP_ENODEV\n"
        "else:\n"
        "    raise SystemExit('quantize ran without a device')\n"
        "assert (q == 0).all()\n"
        "print('ok')\n"
    )
    env = dict(os.environ, PKTITO_HIP_DISABLE="1", PYTHONPATH=ROOT)
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


def test_strerror_names_every_code(so):
    import libpktito_amd as pk
    l = pk.lib()
    names = {c: l.pk_hip_strerror(c).decode() for c in range(7)}
    assert len(set(names.values())) == 7 and names[0] == "ok"
    assert l.pk_hip_strerror(99).decode() == "unknown error"


def test_missing_library_raises(tmp_path, monkeypatch):
    import libpktito_amd as pk
    monkeypatch.setattr(pk, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(pk, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        pk.lib()


REF = "/root/reference"


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "backend", "kernels.h")),
                    reason="the reference checkout is not here")
@pytest.mark.parametrize("src", ["kernels.c", "model_upload.c"])
def test_drop_in_compiles_against_the_reference(src, tmp_path):
    """The backend table and the model-load step, compiled as C11 with the
    reference's own flags against its headers (backend/kernels.h, core/model.h),
    as they would be in backend/hip/ and core/."""
    path = os.path.join(ROOT, "libpktito_amd", "backend_hip", src)
    cmd = ["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fno-math-errno", "-Wall", "-Wextra", "-Werror",
           "-Wpedantic", "-D_DEFAULT_SOURCE", "-D_POSIX_C_SOURCE=200809L",
           "-I", os.path.join(REF, "backend"), "-I", os.path.join(REF, "core"), "-I", os.path.join(ROOT, "include"),
           "-c", path, "-o", str(tmp_path / (src + ".o"))]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    syms = subprocess.run(["nm", str(tmp_path / (src + ".o"))], capture_output=True, text=True).stdout
    if src == "kernels.c":
        assert " R pk_kernels_hip" in syms or " D pk_kernels_hip" in syms
        assert "U pk_hip_gemm_q8" in syms and "U pk_hip_quantize" in syms
    else:
        assert " T pk_hip_upload_model" in syms and " T pk_hip_release_model" in syms
