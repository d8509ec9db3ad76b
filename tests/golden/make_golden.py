"""Cut the golden fixtures from the reference's own compiled ref backend.

    make -C oracle && python tests/golden/make_golden.py

Runs in the container that holds the reference checkout: oracle/Makefile
compiles the reference's backend/ref/kernels.c (with its flags) into
oracle/_ref/libpkref.so, and this script runs that scalar ref - the
reference's definition of correct (backend/kernels.h:9-14) - on the seeded
cases of tests/cases.py, writing what it returns:

    quant.npz    q and d of every quantize case
    gemm.npz     the outputs of every gemm_q8 case (the whole output buffer,
                 the floats between columns included)
    manifest.json  each case's parameters and digests of its inputs and of
                 the activations ref quantized them to

The inputs are regenerated from the seeds (synth.Counter: integer arithmetic
only), and the digests prove a regeneration is the same bytes. The fixtures
are data only; no source of the reference is copied.
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

import cases  # noqa: E402
import oracle_lib as ol  # noqa: E402


def main():
    if ol.ref() is None:
        sys.exit("oracle/_ref/libpkref.so is not built: make -C oracle (needs the reference checkout)")
    manifest = {"source": "peterheb/libpktito backend/ref/kernels.c, compiled by oracle/Makefile",
                "quant": [], "gemm": []}
    qarr = {}
    for name, x, T, n, qb, xs in cases.golden_quant_cases():
        q, d = ol.quantize(x, T, n, qb, xs, impl="ref")
        qarr[f"{name}_q"] = q
        qarr[f"{name}_d"] = d
        manifest["quant"].append(dict(name=name, T=T, n=n, qb=qb, xs=xs, x=cases.digest(x)))
    garr = {}
    for g in cases.golden_gemm_cases():
        n, T, qb = g["n"], g["T"], g["qb"]
        if "q" not in g:
            g["q"], g["d"] = ol.quantize(g["x"], T, n, qb, n, impl="ref")
        out = g["out0"].copy()
        ol.gemm_q8(out, g["os"], g["w"], g["ws"], g["bias"], g["rows"] - g["r0"], g["q"], g["d"],
                   n, qb, T, g["add"], impl="ref", r0=g["r0"])
        garr[g["name"]] = out
        m = {k: g[k] for k in ("name", "rows", "n", "T", "qb", "add", "r0", "os")}
        m["bias"] = g["bias"] is not None
        m["inputs"] = cases.digest(g["w"], g["ws"], g["bias"], g.get("x"), g["out0"])
        m["act"] = cases.digest(g["q"], g["d"])
        for k in ("seed", "pad"):
            if k in g:
                m[k] = g[k]
        manifest["gemm"].append(m)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), **qarr)
    np.savez_compressed(os.path.join(HERE, "gemm.npz"), **garr)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(f"{len(manifest['quant'])} quantize and {len(manifest['gemm'])} gemm_q8 fixtures")


if __name__ == "__main__":
    main()
