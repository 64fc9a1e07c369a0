"""Generates tests/golden/golden.npz: known-answer vectors for the bit-exact
parts of the path (sign words, fp16 scales, INT4 codes, popcounts, binary
scores, entropies).

The reference ships no golden vectors, known-answer tests or fixtures, and
cannot be built here (CUDA only).  The expected outputs below therefore come
from the scalar C oracle (oracle/bitcache_oracle.c, a literal simulation of the
reference kernels' 128-thread blocks) and are cross-checked against the numpy
oracle (oracle/oracle.py) before being written; hand-derived known answers are
asserted separately in tests/test_oracle.py.

Run:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import c_oracle as C  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def special_rows(d: int) -> np.ndarray:
    rows = []
    rows.append(np.full(d, 0.5, np.float16))                       # all positive, constant |x|
    rows.append(np.full(d, -0.25, np.float16))                     # all negative
    alt = np.where(np.arange(d) % 2 == 0, 1.0, -1.0).astype(np.float16)
    rows.append(alt)                                                 # 0x55555555 words
    z = np.zeros(d, np.float16)
    z[1::2] = np.float16(-0.0)
    rows.append(z)                                                   # +-0 -> bits 1, scale 0
    ramp = (np.arange(d) - d / 2).astype(np.float16) / np.float16(8)
    rows.append(ramp)
    big = np.full(d, 60000.0, np.float16)
    big[::3] = -60000.0
    rows.append(big)                                                 # residual absmax overflows fp16
    tiny = np.full(d, 2.0 ** -24, np.float16)
    tiny[::2] = -(2.0 ** -24)
    rows.append(tiny)                                                # subnormal inputs
    sp = np.linspace(-1, 1, d).astype(np.float16)
    sp[0], sp[1], sp[2] = np.inf, -np.inf, np.nan
    rows.append(sp)                                                  # inf / nan handling
    return np.stack(rows)


def main():
    rng = np.random.default_rng(20240601)
    data = {}
    for d in (32, 64, 128, 256):
        x = (rng.standard_normal((48, d)) * rng.lognormal(0, 1.5, (48, 1))).astype(np.float16)
        x = np.concatenate([special_rows(d), x])
        w, s, m = C.binary_encode(x)
        codes2, rs2 = C.residual_encode(x, w, s.astype(np.float32))
        codes1, rs1 = C.residual_encode(x, w, m)
        # cross-check against the numpy oracle before writing
        b = O.binary_encode(x)
        r = O.residual_encode(x, b)
        _, ro = O.online_encode(x)
        assert np.array_equal(b.words, w) and np.array_equal(b.scale.view(np.uint16), s.view(np.uint16))
        assert np.array_equal(r.codes, codes2) and np.array_equal(r.scale.view(np.uint16), rs2.view(np.uint16))
        assert np.array_equal(ro.codes, codes1) and np.array_equal(ro.scale.view(np.uint16), rs1.view(np.uint16))
        data[f"enc_d{d}_x"] = x
        data[f"enc_d{d}_words"] = w
        data[f"enc_d{d}_scale"] = s.view(np.uint16)
        data[f"enc_d{d}_codes"] = codes2
        data[f"enc_d{d}_rscale"] = rs2.view(np.uint16)
        data[f"enc_d{d}_codes_online"] = codes1
        data[f"enc_d{d}_rscale_online"] = rs1.view(np.uint16)

        # query prep + scores for 3 queries x 40 keys
        q = (rng.standard_normal((3, d)) * 0.3).astype(np.float16)
        qw, sq = C.query_prep(q)
        qwt, sqt = C.query_prep(q, tree=True)
        kx = (rng.standard_normal((40, d)) * 0.2).astype(np.float16)
        kw, ks, _ = C.binary_encode(kx)
        pcs, xds, ents = [], [], []
        for i in range(3):
            pc, xd = C.xnor_scores(qw[i], sq[i], kw, ks, d)
            _, xdt = C.xnor_scores(qwt[i], sqt[i], kw, ks, d)
            pcs.append(pc)
            xds.append(xd)
            ents.append(C.entropy(xdt))
        data[f"qs_d{d}_q"] = q
        data[f"qs_d{d}_k"] = kx
        data[f"qs_d{d}_qwords"] = qw
        data[f"qs_d{d}_scale_q"] = sq
        data[f"qs_d{d}_scale_q_tree"] = sqt
        data[f"qs_d{d}_pc"] = np.stack(pcs)
        data[f"qs_d{d}_xdot"] = np.stack(xds)
        data[f"qs_d{d}_entropy"] = np.array(ents, np.float32)
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
