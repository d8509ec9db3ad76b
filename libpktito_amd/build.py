"""Builds libpkhip.so, the C-ABI library of the int8 product path, in-tree.

    python -m libpktito_amd.build        (or libpktito_amd.build.build())

hipcc for gfx950, each source compiled apart (in parallel) and linked into one
shared library: the kernels (csrc/q8_kernels.hip, the quantizer, repack and
products; csrc/layer_kernels.hip, the device-resident layer's float kernels;
csrc/dec_kernels.hip, the decoder's fused per-token launches) and the runtime
(csrc/pk_hip.cpp). The flags are part of the path's contract:
  -ffp-contract=off    no multiply and add the code writes apart is fused: the
                       epilogue's operations are the reference's, one rounding
                       each (its Makefile builds with the same flag);
  no -ffast-math, no -fgpu-flush-denormals-to-zero: a block's scale can be
                       subnormal, and the division must stay IEEE;
  -Xclang -target-feature -Xclang -packed-fp32-ops
                       the packed-fp32 feature off: the compiler makes no
                       v_pk_*_f32 from the epilogue's float code;
  -mllvm --amdgpu-mfma-vgpr-form
                       MFMA accumulators in ordinary VGPRs wherever a kernel
                       fits them: left to its heuristics the register
                       allocator splits the accumulators between VGPRs and
                       AGPRs and copies them around every MFMA of the main
                       loop (three moves an MFMA in the 128 x 128 tile).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libpkhip.so")
SOURCES = [os.path.join(HERE, "csrc", n)
           for n in ("q8_kernels.hip", "q8_stream.hip", "layer_kernels.hip", "dec_kernels.hip", "diag_kernels.hip", "pk_hip.cpp")]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "--amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-result",
]
def flags_for(src):
    """hipcc flags (without -shared) for one source of the library."""
    return [x for x in FLAGS if x != "-shared"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise subprocess.CalledProcessError(r.returncode, cmd, output=out)
    return out


def build(verbose=False):
    """Compile libpkhip.so; raises CalledProcessError with hipcc's output on failure."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc")]
    with tempfile.TemporaryDirectory(prefix="pkhip-") as tmp:
        objs = [os.path.join(tmp, os.path.basename(src) + ".o") for src in SOURCES]
        cmds = [[HIPCC] + flags_for(src) + inc + ["-c", src, "-o", obj] for src, obj in zip(SOURCES, objs)]
        with ThreadPoolExecutor(min(len(cmds), max(1, os.cpu_count() or 1))) as pool:
            outs = list(pool.map(_run, cmds))
        outs.append(_run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", LIB + ".tmp"]))
    out = "\n".join(o for o in outs if o.strip())
    if verbose and out.strip():
        print(out)
    os.replace(LIB + ".tmp", LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
