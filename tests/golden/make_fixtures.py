"""Writes tests/golden/fc_small.npz: a small fully connected LUT case with its
expected lookup indices, min margins, forward output, input gradient and
weight gradient, computed by a plain numpy restatement of the reference's CPU
semantics (index: lut_runtime_kernels_logic.proto:1099-1158; forward blocks:
proto:1214-1299; propagate: proto:1421-1499; weight gradient: proto:1547-1585).
It does not use the C oracle, so the oracle is checked against it.

Run: python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from test_oracle_pins import np_check_detectors, np_du, np_forward  # noqa: E402


def main():
    rng = np.random.default_rng(20240601)
    B, I, T, Nc, O, dgs, ogs = 6, 30, 40, 5, 12, 8, 5
    E = 1 << Nc
    x = rng.random((B, I), dtype=np.float32)
    anchors = np.stack([rng.choice(I, 2, replace=False) for _ in range(T * Nc)]).astype(np.int32).reshape(-1)
    W = (rng.standard_normal(T * E * O) * 0.01).astype(np.float32)
    g = rng.standard_normal((B, O)).astype(np.float32)
    idx, md, mi = np_check_detectors(x, anchors, Nc)
    out = np_forward(W, idx, E, O, dgs)
    # propagate, serial order b -> t -> output block, float += double
    Wr = W.reshape(T, E, O)
    ap = anchors.reshape(T, Nc, 2)
    xg = np.zeros((B, I), np.float32)
    for b in range(B):
        for t in range(T):
            k = mi[b, t]
            for o0 in range(0, O, ogs):
                ms = 0.0
                as_ = 0.0
                for o in range(o0, min(o0 + ogs, O)):
                    gg = float(g[b, o])
                    ms += float(Wr[t, idx[b, t], o]) * gg
                    as_ += float(Wr[t, idx[b, t] ^ (1 << k), o]) * gg
                du = np_du(md[b, t]) * (ms - as_)
                if abs(du) > 1e-17:
                    xg[b, ap[t, k, 0]] = np.float32(float(xg[b, ap[t, k, 0]]) + du)
                    xg[b, ap[t, k, 1]] = np.float32(float(xg[b, ap[t, k, 1]]) - du)
    wg = np.zeros((T, E, O), np.float32)
    for b in range(B):
        for t in range(T):
            for o in range(O):
                if abs(float(g[b, o])) > 1e-17:
                    wg[t, idx[b, t], o] = np.float32(wg[t, idx[b, t], o] + np.float32(float(g[b, o]) * 1.0))
    np.savez_compressed(os.path.join(HERE, "fc_small.npz"), shape=np.array([B, I, T, Nc, O]),
                        dgs=dgs, ogs=ogs, x=x.reshape(-1), anchors=anchors, W=W, g=g.reshape(-1),
                        idx=idx.reshape(-1), md=md.reshape(-1), mi=mi.reshape(-1),
                        out=out.reshape(-1), x_grad=xg.reshape(-1), w_grad=wg.reshape(-1))


if __name__ == "__main__":
    main()
