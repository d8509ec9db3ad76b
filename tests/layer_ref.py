"""Shared by the layer tests: random layer weights in the oracle's dict
form, the positions' activations, the attention composed from a backend's
float kernels, and the packed activations' layout read back. Test
infrastructure."""
import numpy as np

import oracle_lib as ol
from libpktito_amd import synth
from libpktito_amd.synth import layer_weights  # noqa: F401  (the tests' import point)


def positions(g, T, D, qb):
    ape = g.standard_normal((2 * T - 1, D)).astype(np.float32)
    q, d = ol.quantize(ape.reshape(-1), 2 * T - 1, D, qb, D)
    return ape, q, d


def attention(q, k, v, p, bias_u, bias_v, H, impl="oracle"):
    """core/encoder.c:280-327 from a backend's pk_k_gemm_f32 and pk_k_softmax
    (the oracle's, or the reference's with impl="ref"), with the operands laid
    out here by numpy as that kernel's panels: o [T, D] from q, k, v [T, D]
    and the positions' p [2T - 1, D]."""
    T, D = q.shape
    R, dk = 2 * T - 1, D // H
    scale = np.float32(1.0) / np.sqrt(np.float32(dk))
    o = np.zeros((T, D), np.float32)

    def panels(m, rows):
        # 16 rows a panel, k-major: W(d, j) at ((j / 16) dk + d) 16 + j % 16
        pad = np.zeros(((rows + 15) // 16 * 16, dk), np.float32)
        pad[:rows] = m
        return pad.reshape(-1, 16, dk).transpose(0, 2, 1).reshape(-1)

    for h in range(H):
        hs = slice(h * dk, (h + 1) * dk)
        qu = (q[:, hs] + bias_u[hs]).astype(np.float32)
        qv = (q[:, hs] + bias_v[hs]).astype(np.float32)
        sc = ol.gemm_f32(panels(k[:, hs], T), dk, (T + 15) // 16 * 16, dk, qu, T, impl=impl)[:, :T]
        bd = ol.gemm_f32(panels(p[:, hs], R), dk, (R + 15) // 16 * 16, dk, qv, T, impl=impl)
        s = np.empty((T, T), np.float32)
        for i in range(T):
            s[i] = sc[i] + bd[i, T - 1 - i:2 * T - 1 - i]
        s = ol.softmax(s, scale, impl=impl)
        # values as panels of 16 dimensions, key-major
        vp = np.ascontiguousarray(v[:, hs].T).reshape(dk // 16, 16, T).transpose(0, 2, 1).reshape(-1)
        o[:, hs] = ol.gemm_f32(vp, T, dk, T, s, T, impl=impl)
    return o


def unpack_packed(qp, n, T):
    """Packed activations (16-frame groups, units of 16 x 64 in MFMA order,
    stage-major) back to row-major [T, n]."""
    G = (T + 15) // 16
    ku = len(qp) // (G * 1024)
    u = qp.reshape(ku, G, 4, 16, 16)            # [unit][group][kq][row][16 bytes]
    full = u.transpose(1, 3, 0, 2, 4).reshape(G * 16, ku * 64)
    return full[:T, :n]
