"""Pins the CPU oracle (oracle/lut_oracle.c) against what the mathematics fixes,
independently of the oracle's own code: brute force on tiny inputs, closed
forms with exactly representable values, special cases, and checks built so
that a plausible mistake (dropped term, swapped operand, wrong bit order,
wrong rounding point) fails.

The reference ships no golden vectors for the LUT path (its tests are
differential, src/spiky/lut/tests/); the committed fixtures under
tests/golden/ are produced by tests/golden/make_fixtures.py from the plain
numpy restatement below and checked here too.
"""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


# ---------------------------------------------------------------- numpy restatement
def np_check_detectors(x, anchors, n_anchors, cmp_eps=0.0):
    """Textbook index: bit k set iff x[a1]-x[a2] > 0 (outside the +-eps band);
    min margin = first k with strictly smallest |delta| (gt_lut_transformer.py
    LUT.cache_index semantics, lut_runtime_kernels_logic.proto:1137-1148)."""
    B = x.shape[0]
    T = anchors.shape[0] // (2 * n_anchors)
    ap = anchors.reshape(T, n_anchors, 2)
    idx = np.zeros((B, T), np.int32)
    md = np.zeros((B, T), np.float32)
    mi = np.full((B, T), -1, np.int32)
    for b in range(B):
        for t in range(T):
            best = None
            for k in range(n_anchors):
                a1, a2 = ap[t, k]
                if a1 < 0 or a2 < 0:
                    continue
                d = np.float32(x[b, a1]) - np.float32(x[b, a2])
                bit = (d > 0) if cmp_eps == 0 else (False if abs(d) < cmp_eps else d > 0)
                if bit:
                    idx[b, t] |= 1 << k
                if best is None or abs(d) < abs(best):
                    best = d
                    md[b, t] = d
                    mi[b, t] = k
    return idx, md, mi


def np_forward(W, idx, E, O, dgs):
    """out[b,o] = sum over blocks of fp32(fp64 sum of the block's rows)."""
    B, T = idx.shape
    Wr = W.reshape(T, E, O).astype(np.float64)
    out = np.zeros((B, O), np.float32)
    for b in range(B):
        for t0 in range(0, T, dgs):
            s = np.zeros(O, np.float64)
            for t in range(t0, min(t0 + dgs, T)):
                s = s + Wr[t, idx[b, t]]
            out[b] = out[b] + s.astype(np.float32)
    return out


def np_du(md):
    u = np.float64(md)
    r = 1.0 / (1.0 + abs(u))
    return r * (0.5 * r) if u > 0 else r * (-0.5 * r)


# ---------------------------------------------------------------- check_detectors
def test_check_detectors_brute_force(oracle):
    rng = np.random.default_rng(0)
    B, I, T, Nc = 5, 12, 9, 4
    x = rng.integers(-3, 4, size=(B, I)).astype(np.float32)  # many exact ties and zeros
    anchors = np.stack([rng.choice(I, 2, replace=False) for _ in range(T * Nc)]).astype(np.int32).reshape(-1)
    idx, md, mi = oracle.check_detectors(x.reshape(-1), anchors, B, I, T, Nc)
    ridx, rmd, rmi = np_check_detectors(x, anchors, Nc)
    assert np.array_equal(idx.reshape(B, T), ridx)
    assert np.array_equal(md.reshape(B, T), rmd)
    assert np.array_equal(mi.reshape(B, T), rmi)


def test_check_detectors_special_cases(oracle):
    # one detector, 3 anchors: delta = 0 -> bit 0; tie of |delta| -> lowest k kept
    x = np.array([[1.0, 1.0, 3.0, 2.0, 0.0]], np.float32)
    anchors = np.array([0, 1, 2, 3, 3, 2], np.int32)  # deltas 0, +1, -1
    idx, md, mi = oracle.check_detectors(x.reshape(-1), anchors, 1, 5, 1, 3)
    assert idx[0] == 0b010 and md[0] == 0.0 and mi[0] == 0
    # no zero: deltas +1, -1 -> tie on |1|, first wins with its sign
    anchors = np.array([2, 3, 3, 2, 2, 4], np.int32)  # +1, -1, +3
    idx, md, mi = oracle.check_detectors(x.reshape(-1), anchors, 1, 5, 1, 3)
    assert idx[0] == 0b101 and md[0] == 1.0 and mi[0] == 0
    # unused pair (-1) is skipped, bit stays 0, never the min
    anchors = np.array([-1, -1, 3, 2, 2, 4], np.int32)
    idx, md, mi = oracle.check_detectors(x.reshape(-1), anchors, 1, 5, 1, 3)
    assert idx[0] == 0b100 and md[0] == -1.0 and mi[0] == 1
    # cmp_eps band: |delta| < eps gives bit 0
    anchors = np.array([2, 3, 3, 4, 0, 4], np.int32)  # +1, +2, +1
    idx = oracle.check_detectors(x.reshape(-1), anchors, 1, 5, 1, 3, cmp_eps=1.5, train=False)
    assert idx[0] == 0b010
    # NaN: a NaN first anchor stays the min (|NaN| < m is always false)
    xn = np.array([[np.nan, 1.0, 3.0, 2.0]], np.float32)
    anchors = np.array([0, 1, 2, 3], np.int32)
    idx, md, mi = oracle.check_detectors(xn.reshape(-1), anchors, 1, 4, 1, 2)
    assert idx[0] == 0b10 and np.isnan(md[0]) and mi[0] == 0


# ---------------------------------------------------------------- forward
def _rand_case(rng, B, I, T, Nc, O):
    E = 1 << Nc
    x = rng.random((B, I), dtype=np.float32)
    anchors = np.stack([rng.choice(I, 2, replace=False) for _ in range(T * Nc)]).astype(np.int32).reshape(-1)
    W = (rng.standard_normal(T * E * O) * 0.01).astype(np.float32)
    return x, anchors, W, E


def test_forward_exact_integers(oracle):
    """Integer weights: every fp64/fp32 step is exact, so the result is the plain gather-sum."""
    rng = np.random.default_rng(1)
    B, T, Nc, O = 4, 70, 3, 5
    E = 1 << Nc
    W = rng.integers(-50, 50, size=T * E * O).astype(np.float32)
    idx = rng.integers(0, E, size=(B, T)).astype(np.int32)
    out = oracle.fill_outputs_fc(W, idx, B, O, T, E, dgs=32).reshape(B, O)
    ref = W.reshape(T, E, O)[np.arange(T)[None, :], idx].sum(axis=1)
    assert np.array_equal(out, ref.astype(np.float32))


def test_forward_block_rounding_points(oracle):
    """fp64 within a block, one fp32 commit per block: 1e8+1 rounds to 1e8 in fp32,
    so blocks {1e8, 1}, {-1e8, 1} give 0, while a plain fp64 sum gives 2 and a
    plain fp32 running sum gives 1."""
    W = np.array([1e8, 1.0, -1e8, 1.0], np.float32)  # T=4 detectors, E=1, O=1
    idx = np.zeros((1, 4), np.int32)
    out = oracle.fill_outputs_fc(W, idx, 1, 1, 4, 1, dgs=2)
    assert out[0] == 0.0
    assert np_forward(W, idx, 1, 1, 2)[0, 0] == 0.0
    assert oracle.fill_outputs_fc(W, idx, 1, 1, 4, 1, dgs=1)[0] == 1.0
    assert oracle.fill_outputs_fc(W, idx, 1, 1, 4, 1, dgs=4)[0] == 2.0


def test_forward_matches_numpy_random(oracle):
    rng = np.random.default_rng(2)
    B, I, T, Nc, O = 3, 40, 45, 4, 7
    x, anchors, W, E = _rand_case(rng, B, I, T, Nc, O)
    idx = oracle.check_detectors(x.reshape(-1), anchors, B, I, T, Nc, train=False)
    out = oracle.fill_outputs_fc(W, idx, B, O, T, E, dgs=8).reshape(B, O)
    ref = np_forward(W, idx.reshape(B, T), E, O, 8)
    assert np.array_equal(out, ref)
    # a transposed table layout ([E][T][O]) would not match
    Wt = W.reshape(T, E, O).transpose(1, 0, 2).copy().reshape(-1)
    assert not np.array_equal(np_forward(Wt, idx.reshape(B, T), E, O, 8), ref)


def test_forward_int_mode_closed_form(oracle):
    """int32 payload per block = trunc(sum * 1048575 * rescaler); epilogue
    (acc * 9.536752259018191e-07) / rescaler."""
    W = np.array([0.25, 0.5, -0.125, 0.375], np.float32)  # T=4, E=1, O=1
    idx = np.zeros((1, 4), np.int32)
    resc = 0.5
    acc = oracle.fill_outputs_fc(W, idx, 1, 1, 4, 1, dgs=2, int_mode=True, int_rescaler=resc)
    p1 = int(np.trunc((0.25 + 0.5) * 1048575.0 * resc))
    p2 = int(np.trunc((-0.125 + 0.375) * 1048575.0 * resc))
    assert acc.view(np.int32)[0] == p1 + p2
    oracle.convert_int_to_float(acc, resc)
    assert acc[0] == np.float32(((p1 + p2) * 9.536752259018191e-07) / resc)


def test_forward_int8_dequant(oracle):
    rng = np.random.default_rng(3)
    B, T, Nc, O = 2, 33, 2, 4
    E = 1 << Nc
    q = rng.integers(-127, 128, size=T * E * O).astype(np.int8)
    sc = rng.uniform(0.001, 0.01, size=T).astype(np.float32)
    idx = rng.integers(0, E, size=(B, T)).astype(np.int32)
    out = oracle.fill_outputs_fc(None, idx, B, O, T, E, dgs=32, q8=q, scales=sc)
    Wd = (sc[:, None] * q.reshape(T, E * O).astype(np.float32)).astype(np.float32).reshape(-1)
    assert np.array_equal(out.reshape(B, O), np_forward(Wd, idx, E, O, 32))


# ---------------------------------------------------------------- backward
def test_propagate_textbook_single_block(oracle):
    """With O <= ogs there is one dot per (b, t): the textbook LUT backward
    (gt_lut_transformer.py LUT.backward): du = sign(u) 0.5/(1+|u|)^2 *
    g.(W_main - W_alt); x[a1] += du, x[a2] -= du."""
    rng = np.random.default_rng(4)
    B, I, T, Nc, O = 3, 10, 6, 3, 5
    x, anchors, W, E = _rand_case(rng, B, I, T, Nc, O)
    g = rng.standard_normal((B, O)).astype(np.float32)
    idx, md, mi = oracle.check_detectors(x.reshape(-1), anchors, B, I, T, Nc)
    xg = oracle.propagate_fc(W, g, idx, md, mi, anchors, B, I, O, T, Nc, E, ogs=32).reshape(B, I)
    ref = np.zeros((B, I), np.float64)
    Wr = W.reshape(T, E, O).astype(np.float64)
    ap = anchors.reshape(T, Nc, 2)
    idx, md, mi = idx.reshape(B, T), md.reshape(B, T), mi.reshape(B, T)
    for b in range(B):
        for t in range(T):
            k = mi[b, t]
            du = np_du(md[b, t]) * (g[b].astype(np.float64) @ (Wr[t, idx[b, t]] - Wr[t, idx[b, t] ^ (1 << k)]))
            ref[b, ap[t, k, 0]] += du
            ref[b, ap[t, k, 1]] -= du
    np.testing.assert_allclose(xg, ref, rtol=1e-6, atol=1e-9)
    # swapping main and alt rows flips every contribution
    assert not np.allclose(xg, -ref, rtol=1e-3, atol=1e-9)


def test_propagate_block_split(oracle):
    """Splitting the outputs into blocks of ogs changes nothing but rounding:
    the sum over blocks equals the single-block result."""
    rng = np.random.default_rng(5)
    B, I, T, Nc, O = 2, 16, 9, 4, 37
    x, anchors, W, E = _rand_case(rng, B, I, T, Nc, O)
    g = rng.standard_normal((B, O)).astype(np.float32)
    idx, md, mi = oracle.check_detectors(x.reshape(-1), anchors, B, I, T, Nc)
    a = oracle.propagate_fc(W, g, idx, md, mi, anchors, B, I, O, T, Nc, E, ogs=64)
    b = oracle.propagate_fc(W, g, idx, md, mi, anchors, B, I, O, T, Nc, E, ogs=4)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-7)


def test_wgrad_brute_force(oracle):
    """w_grad[t, idx[b,t], :] += lr * g[b, :] in ascending b; integer-valued g
    makes the fp32 sums exact, so it equals np.add.at."""
    rng = np.random.default_rng(6)
    B, T, Nc, O = 9, 7, 2, 6
    E = 1 << Nc
    g = rng.integers(-8, 9, size=(B, O)).astype(np.float32)
    idx = rng.integers(0, E, size=(B, T)).astype(np.int32)
    wg = np.zeros(T * E * O, np.float32)
    oracle.gather_wgrad_fc(g, idx, wg, B, O, T, E, ogs=4, first_meta_lr=0.5)
    ref = np.zeros((T, E, O), np.float64)
    for b in range(B):
        for t in range(T):
            ref[t, idx[b, t]] += 0.5 * g[b]
    assert np.array_equal(wg.reshape(T, E, O), ref.astype(np.float32))
    # Internal policy: the update is -lr*external_lr*g applied to the weights
    W = np.ones(T * E * O, np.float32)
    oracle.gather_wgrad_fc(g, idx, W, B, O, T, E, ogs=4, first_meta_lr=0.5, external_lr=0.25)
    assert np.array_equal(W.reshape(T, E, O), (1.0 - 0.25 * ref).astype(np.float32))


def test_wgrad_eps_skip(oracle):
    """|g| <= 1e-17 contributes nothing (gather_weight_gradients_fc, proto:792-818)."""
    g = np.array([[1e-18, -1e-17, 2e-17]], np.float32)
    idx = np.zeros((1, 1), np.int32)
    wg = np.zeros(3, np.float32)
    oracle.gather_wgrad_fc(g, idx, wg, 1, 3, 1, 1)
    assert wg[0] == 0 and wg[1] == 0 and wg[2] == np.float32(2e-17)


# ---------------------------------------------------------------- anchors
def test_decode_compact_is_bijection(oracle):
    """Codes 0..n(n-1)-1 map one-to-one onto ordered pairs (a1 != a2) of the
    detector's input list, in lexicographic order."""
    n = 6
    ids = np.array([3, 8, 11, 20, 21, 40], np.int32)
    codes = np.arange(n * (n - 1), dtype=np.int64)
    anchors, err = oracle.decode_anchors_compact(codes, 1, n * (n - 1), n * (n - 1),
                                                 np.array([0, n], np.int64), ids)
    assert err == 0
    pairs = anchors.reshape(n * (n - 1), 2)
    expect = [(ids[a], ids[b]) for a in range(n) for b in range(n) if a != b]
    assert [tuple(p) for p in pairs] == expect


def test_decode_compact_errors(oracle):
    codes = np.zeros(4, np.int64)
    anchors, err = oracle.decode_anchors_compact(codes, 2, 2, 2, np.array([0, 1, 3], np.int64),
                                                 np.array([5, 6, 7], np.int32))
    assert err == 1  # first detector has a single input


# ---------------------------------------------------------------- sparse == FC
def test_sparse_equals_fc_when_fully_connected(oracle):
    """A sparse layer whose every lookup neuron targets all outputs in order is
    the FC layer (the reference's own equivalence test,
    test_lut_fully_connected_small.py:29-139): forward exact for integer
    weights; propagate and w_grad bit-identical when groups = output blocks."""
    rng = np.random.default_rng(7)
    B, I, T, Nc, O, ogs = 3, 12, 10, 3, 9, 4
    x, anchors, W, E = _rand_case(rng, B, I, T, Nc, O)
    g = rng.standard_normal((B, O)).astype(np.float32)
    offs = np.arange(T * E + 1, dtype=np.int64) * O
    tg = np.tile(np.arange(O, dtype=np.int32), T * E)
    idx, md, mi = oracle.check_detectors(x.reshape(-1), anchors, B, I, T, Nc)
    Wi = rng.integers(-20, 20, size=W.size).astype(np.float32)
    f1 = oracle.fill_outputs_fc(Wi, idx, B, O, T, E, dgs=4)
    f2 = oracle.fill_outputs_sparse(Wi, idx, offs, tg, B, O, T, E)
    assert np.array_equal(f1, f2)
    p1 = oracle.propagate_fc(W, g, idx, md, mi, anchors, B, I, O, T, Nc, E, ogs=ogs)
    p2 = oracle.propagate_sparse(W, g, idx, md, mi, anchors, offs, tg, B, I, O, T, Nc, E, ogs,
                                 (O + ogs - 1) // ogs)
    assert np.array_equal(p1, p2)
    w1 = np.zeros(W.size, np.float32)
    w2 = np.zeros(W.size, np.float32)
    oracle.gather_wgrad_fc(g, idx, w1, B, O, T, E, ogs=ogs)
    oracle.gather_wgrad_sparse(g, idx, offs, tg, w2, B, O, T, E)
    assert np.array_equal(w1, w2)


# ---------------------------------------------------------------- golden fixtures
def test_golden_fixtures(oracle):
    path = os.path.join(HERE, "golden", "fc_small.npz")
    if not os.path.exists(path):
        pytest.skip("fixtures not generated")
    z = np.load(path)
    B, I, T, Nc, O = (int(v) for v in z["shape"])
    E = 1 << Nc
    idx, md, mi = oracle.check_detectors(z["x"], z["anchors"], B, I, T, Nc)
    assert np.array_equal(idx, z["idx"]) and np.array_equal(md, z["md"]) and np.array_equal(mi, z["mi"])
    out = oracle.fill_outputs_fc(z["W"], idx, B, O, T, E, dgs=int(z["dgs"]))
    assert np.array_equal(out, z["out"])
    xg = oracle.propagate_fc(z["W"], z["g"], idx, md, mi, z["anchors"], B, I, O, T, Nc, E,
                             ogs=int(z["ogs"]))
    np.testing.assert_allclose(xg, z["x_grad"], rtol=1e-5, atol=1e-8)
    wg = np.zeros(T * E * O, np.float32)
    oracle.gather_wgrad_fc(z["g"], idx, wg, B, O, T, E, ogs=int(z["ogs"]))
    assert np.array_equal(wg, z["w_grad"])


def test_dense_to_sparse_oracle_pins(oracle):
    """The converter's selection rule, pinned by the reference docstring's
    example (torch_utils.py:14-20), the bit-pattern rule of its int4 compare
    (a float -0.0 is kept, torch_utils_kernels_logic.proto:20-35), int32
    words, and a brute-force loop on a random array."""
    idx, val = oracle.dense_to_sparse_32(np.array([1.0, 0.0, 2.0, 0.0, 3.0], np.float32))
    assert idx.tolist() == [0, 2, 4] and val.tolist() == [1.0, 2.0, 3.0]
    idx, val = oracle.dense_to_sparse_32(np.array([0.0, -0.0, 0.0, 5.0], np.float32))
    assert idx.tolist() == [1, 3]
    assert np.signbit(val[0]) and val[0] == 0.0
    idx, val = oracle.dense_to_sparse_32(np.array([0, -7, 0, (1 << 31) - 1], np.int32))
    assert idx.tolist() == [1, 3] and val.tolist() == [-7, (1 << 31) - 1]
    rng = np.random.default_rng(5)
    a = rng.random(1000).astype(np.float32)
    a[a > 0.5] = 0.0
    a[::37] = -0.0
    want = [i for i in range(a.size) if a.view(np.uint32)[i] != 0]
    idx, val = oracle.dense_to_sparse_32(a)
    assert idx.tolist() == want
    assert np.array_equal(val.view(np.uint32), a.view(np.uint32)[want])
    with pytest.raises(ValueError):
        oracle.dense_to_sparse_32(np.zeros(4, np.float64))
