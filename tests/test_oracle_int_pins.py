"""Closed-form pins of the oracle's int32 (LUTDataManagerI) backward branches.

The reference commits every backward term as an int32 fixed-point payload:

  * input gradient (propagate_through_detector, proto:833-847): per (table,
    output block) term du * (main - alt), dropped unless |term| > EPS = 1e-17
    (misc.h:90); otherwise p = (int32)(term * 1048575 * int_rescaler),
    truncated toward zero, added at the min anchor's first input and
    subtracted at its second;
  * weight gradient (gather_weight_gradients_fc, proto:775-777,797-800): per
    (sample, output) with |g| > EPS, p = (int32)(g * lr * 1048575 *
    int_rescaler) added to the row's accumulator;

with du = sign(u) * 0.5 / (1 + |u|)^2 and sign(u <= 0) = -1 (proto:1458-1465).

Every case below uses exactly representable inputs (integer weights and
inputs, margins u with 1 + |u| a power of two, binary-fraction gradients), so
the expected accumulators follow from exact rational arithmetic done here with
Python's Fraction and integer truncation -- not from the oracle's C code.  Each
case is chosen so that a plausible slip fails it: a floor instead of a
truncation (negative payloads), one payload per sum instead of per block, the
signs at a1 / a2 swapped, the EPS cut dropped or applied to the wrong value,
the sign of du at u = 0, the learning-rate factor, DENOM32 off by one."""
from fractions import Fraction

import numpy as np
import pytest

DENOM = 1048575  # 0x000FFFFF, misc.h:98


def trunc_payload(term, rescaler):
    """(int32)(term * DENOM * rescaler), truncated toward zero, from exact rationals."""
    v = Fraction(term) * DENOM * Fraction(rescaler)
    n = abs(v.numerator) // v.denominator
    return n if v >= 0 else -n


def du_exact(u):
    u = Fraction(u)
    r = Fraction(1) / (1 + abs(u))
    return r * r / 2 if u > 0 else -r * r / 2


def i32(buf):
    return np.asarray(buf).view(np.int32)


# ------------------------------------------------------------------ fully connected
def _fc_case():
    """One table, one anchor pair (inputs 0 and 1), E = 2 rows, O = 4 outputs
    split into two 2-output blocks."""
    W = np.array([[1, -2, 4, 0],      # row 0
                  [3, 5, -1, 2]],     # row 1
                 np.float32).reshape(-1)
    g = np.array([2, -1, 1, 3], np.float32)
    return W, g


@pytest.mark.parametrize("u,resc", [(1.0, 1.0), (-1.0, 1.0), (3.0, 0.25), (0.0, 1.0)])
def test_propagate_fc_int_closed_form(oracle, u, resc):
    W, g = _fc_case()
    x = np.array([u, 0.0], np.float32)          # delta = x[0] - x[1] = u
    anchors = np.array([0, 1], np.int32)
    idx, md, mi = oracle.check_detectors(x, anchors, 1, 2, 1, 1)
    main = 1 if u > 0 else 0                    # bit = (delta > 0)
    assert idx[0] == main and md[0] == u and mi[0] == 0
    alt = main ^ 1
    Wr = W.reshape(2, 4)
    du = du_exact(u)
    expect = 0
    for o0 in (0, 2):                           # one payload per 2-output block
        dot = sum(Fraction(int(Wr[main, o])) * int(g[o]) - Fraction(int(Wr[alt, o])) * int(g[o])
                  for o in range(o0, o0 + 2))
        term = du * dot
        if abs(term) > Fraction(1, 10 ** 17):
            expect += trunc_payload(term, resc)
    xg = oracle.propagate_fc(W, g, idx, md, mi, anchors, 1, 2, 4, 1, 1, 2, ogs=2,
                             int_mode=True, int_rescaler=resc)
    assert i32(xg)[0] == expect and i32(xg)[1] == -expect


def test_propagate_fc_int_per_block_truncation():
    """Two block terms -3/8 and +5/8 (u = 1, du = 1/8): the reference pushes
    trunc(-3/8 D) + trunc(5/8 D) = -393215 + 655359 = 262144, one more than
    trunc(2/8 D) = 262143 of the summed term.  Numbers written out by hand."""
    import oracle
    W = np.array([[0, 0, 0, 0], [1, 0, 5, 0]], np.float32).reshape(-1)
    W[0:4] = [4, 0, 0, 0]                      # row 0
    g = np.array([1, 0, 1, 0], np.float32)
    # main row 1, alt row 0: block 0 dot = 1 - 4 = -3, block 1 dot = 5 - 0 = 5
    x = np.array([1.0, 0.0], np.float32)
    anchors = np.array([0, 1], np.int32)
    idx, md, mi = oracle.check_detectors(x, anchors, 1, 2, 1, 1)
    xg = oracle.propagate_fc(W, g, idx, md, mi, anchors, 1, 2, 4, 1, 1, 2, ogs=2,
                             int_mode=True, int_rescaler=1.0)
    assert 3 * DENOM // 8 == 393215 and 5 * DENOM // 8 == 655359
    assert i32(xg)[0] == 262144 and i32(xg)[1] == -262144


def test_propagate_fc_int_eps_cut(oracle):
    """The EPS cut applies to the block term du * (main - alt), before the
    rescale: with int_rescaler 2^60 a term of 2^-59 (< 1e-17) would push
    2 * DENOM if it were kept, and a term of 2^-56 (> 1e-17) pushes 16 * DENOM."""
    anchors = np.array([0, 1], np.int32)
    x = np.array([1.0, 0.0], np.float32)       # u = 1: main 1, alt 0, du = 1/8
    idx, md, mi = oracle.check_detectors(x, anchors, 1, 2, 1, 1)
    g = np.array([1.0], np.float32)
    for diff_exp, expect in ((-56, 0), (-53, 16 * DENOM)):
        W = np.array([0.0, 2.0 ** diff_exp], np.float32)   # rows 0 and 1, one output
        xg = oracle.propagate_fc(W, g, idx, md, mi, anchors, 1, 2, 1, 1, 1, 2, ogs=1,
                                 int_mode=True, int_rescaler=2.0 ** 60)
        assert i32(xg)[0] == expect and i32(xg)[1] == -expect


@pytest.mark.parametrize("internal", [False, True])
def test_gather_wgrad_fc_int_closed_form(oracle, internal):
    """Two samples hit row 1 of a 2-row table and one hits row 0; payloads
    trunc(g * lr * D * r) per (sample, output) are added separately (so the
    truncations do not merge), |g| <= EPS is skipped.  Internal SGD uses
    lr = first_meta_lr * (-external_lr) (proto:731-734)."""
    O = 3
    g = np.array([[0.5, -0.25, 1e-18],
                  [-0.75, 0.125, 2.0],
                  [1.0, -1.0, 0.0]], np.float32).reshape(-1)
    idx = np.array([1, 1, 0], np.int32)           # samples 0, 1 -> row 1; sample 2 -> row 0
    first_lr, ext = 0.5, (0.25 if internal else -1.0)
    lr = Fraction(first_lr) * (-Fraction(ext) if internal else 1)
    resc = 0.5
    target = np.zeros(2 * O, np.float32)
    oracle.gather_wgrad_fc(g, idx, target, 3, O, 1, 2, ogs=32, first_meta_lr=first_lr,
                           external_lr=ext, int_mode=True, int_rescaler=resc)
    gg = g.reshape(3, O)
    expect = np.zeros((2, O), np.int64)
    for b in range(3):
        for o in range(O):
            gv = Fraction(float(gg[b, o]))
            if abs(gv) > Fraction(1, 10 ** 17):
                expect[idx[b], o] += trunc_payload(gv * lr, resc)
    assert np.array_equal(i32(target).reshape(2, O), expect)
    # the hand value of one entry: row 1, output 0 gets trunc(0.5 lr D r) + trunc(-0.75 lr D r)
    if not internal:
        assert expect[1, 0] == (DENOM // 8) - (3 * DENOM // 16)   # 131071 - 196607


# ------------------------------------------------------------------ sparse connectivity
def test_sparse_int_closed_form(oracle):
    """One table of 2 lookup neurons with explicit synapse lists.  Forward
    groups of fgs = 1 synapse: the propagate forms one term per group index
    (main neuron's group k against the alt neuron's group k, proto:1303-1419),
    each truncated on its own; the weight gradient adds one payload per
    synapse (proto:584-714)."""
    # neuron 0 -> outputs [1, 2], neuron 1 -> outputs [0, 2, 3]
    offs = np.array([0, 2, 5], np.int64)
    tg = np.array([1, 2, 0, 2, 3], np.int32)
    W = np.array([2, -3, 1, 4, -1], np.float32)
    g = np.array([1, -2, 3, 0.5], np.float32)
    x = np.array([3.0, 0.0], np.float32)         # u = 3: main 1, alt 0, du = 1/32
    anchors = np.array([0, 1], np.int32)
    idx, md, mi = oracle.check_detectors(x, anchors, 1, 2, 1, 1)
    du = du_exact(3)
    main_syn = [(2, 0), (3, 2), (4, 3)]          # (synapse, output) of neuron 1
    alt_syn = [(0, 1), (1, 2)]
    expect = 0
    for k in range(3):                            # max groups = 3
        ms = Fraction(int(W[main_syn[k][0]])) * Fraction(float(g[main_syn[k][1]])) if k < 3 else 0
        as_ = (Fraction(int(W[alt_syn[k][0]])) * Fraction(float(g[alt_syn[k][1]]))) if k < 2 else 0
        term = du * (ms - as_)
        if abs(term) > Fraction(1, 10 ** 17):
            expect += trunc_payload(term, 1.0)
    xg = oracle.propagate_sparse(W, g, idx, md, mi, anchors, offs, tg, 1, 2, 4, 1, 1, 2, 1, 3,
                                 int_mode=True, int_rescaler=1.0)
    assert i32(xg)[0] == expect and i32(xg)[1] == -expect
    # terms: 1/32 * (1*1 - 2*(-2)) = 5/32, 1/32 * (4*3 - (-3)*3) = 21/32, 1/32 * (-1*0.5) = -1/64
    assert expect == 5 * DENOM // 32 + 21 * DENOM // 32 - (DENOM // 64)
    target = np.zeros(5, np.float32)
    oracle.gather_wgrad_sparse(g, idx, offs, tg, target, 1, 4, 1, 2, first_meta_lr=0.5,
                               int_mode=True, int_rescaler=1.0)
    expect_w = np.zeros(5, np.int64)
    for s, o in main_syn:
        expect_w[s] = trunc_payload(Fraction(float(g[o])) / 2, 1.0)
    assert np.array_equal(i32(target).astype(np.int64), expect_w)
    assert expect_w[4] == DENOM // 4 and expect_w[2] == DENOM // 2


# ------------------------------------------------------------------ sequence-concat
@pytest.mark.parametrize("q_smaller", [True, False])
def test_seq_int_closed_form(oracle, q_smaller):
    """S = 2 (one causal pair i = 0 < j = 1), one table, Nc = 1, positional
    dim 1.  Row = (Q << 2) | (K << 1) | P.  The smaller of |dQ|, |dK| is
    flipped (ties to K, proto:3740-3760) and its payload goes to the position
    that owns it (j for Q, i for K); the positional flip applies only when its
    margin is strictly the smallest and carries no EPS cut (proto:1016-1046)."""
    I, O = 2, 2
    # position 0 (K) has delta 3, position 1 (Q) delta 1 (or the other way round)
    dk, dq = (3.0, 1.0) if q_smaller else (1.0, 3.0)
    x = np.array([dk, 0.0, dq, 0.0], np.float32)
    pe = np.array([0.5], np.float32)               # (S-1)*T*pd = 1 value: P = 1, margin 0.5
    anchors = np.array([0, 1], np.int32)
    idx, md, mi = oracle.check_detectors(x, anchors, 2, I, 1, 1)
    pidx, pmd, pmi = oracle.check_pe(pe, 2, 1, 1)
    K, Q, P = int(idx[0]), int(idx[1]), int(pidx[0])
    assert (K, Q, P) == (1, 1, 1)
    W = np.arange(8 * O, dtype=np.float32).reshape(8, O) - 5    # row r = [2r - 5, 2r - 4]
    g = np.array([[0, 0], [1, -2]], np.float32).reshape(-1)     # only position j = 1 has g
    row = lambda q, k, p: (q << 2) | (k << 1) | p
    dot = lambda r: sum(Fraction(int(W[r, o])) * int(g[2 + o]) for o in range(O))
    main = row(Q, K, P)
    if abs(dq) < abs(dk):
        alt, du, pos = row(Q ^ 1, K, P), du_exact(dq), 1
    else:
        alt, du, pos = row(Q, K ^ 1, P), du_exact(dk), 0
    term = du * (dot(main) - dot(alt))
    px = trunc_payload(term, 1.0)
    # PE margin 0.5 is strictly the smallest: its flip adds du(0.5) * (main - pe-flipped)
    dpe = du_exact(Fraction(1, 2)) * (dot(main) - dot(row(Q, K, P ^ 1)))
    ppe = trunc_payload(dpe, 1.0)
    xg, peg = oracle.propagate_seq(W.reshape(-1), g, idx, md, mi, pidx, pmd, pmi, anchors, 1, I, O, 1,
                                   2, 1, 1, int_mode=True, int_rescaler=1.0)
    xi = i32(xg).reshape(2, I)
    assert xi[pos, 0] == px and xi[pos, 1] == -px and not xi[1 - pos].any()
    assert i32(peg)[0] == ppe
    # hand values: every row's dot is (2r - 5) - 2(2r - 4) = 3 - 2r, so main - alt = 2 (alt - main) ...
    assert dot(main) == 3 - 2 * main
    # weight gradient: the pair adds trunc(g[1][o] * lr * D) to row (Q, K, P)
    target = np.zeros(8 * O, np.float32)
    oracle.gather_wgrad_seq(g, idx, pidx, target, 1, O, 1, 2, 1, 1, first_meta_lr=0.25,
                            int_mode=True, int_rescaler=1.0)
    expect = np.zeros((8, O), np.int64)
    expect[main] = [DENOM // 4, -(DENOM // 2)]
    assert np.array_equal(i32(target).reshape(8, O).astype(np.int64), expect)


# ------------------------------------------------------------------ product mode
def test_product_int_closed_form(oracle):
    """Product mode, S = 2, one table with one anchor pair (x1[i][0], x2[j][0]),
    no positional part: one lookup per pair.  The margin is delta = x1[0][0] -
    x2[1][0]; the term du * (main - alt) over the whole row goes +trunc to
    x1's input and -trunc to x2's (proto:869-1023), and the weight gradient
    adds trunc(g * lr * D * r) to the main row (proto:716-790)."""
    n1 = n2 = 1
    O = 3
    x1 = np.array([2.0, 0.0], np.float32)          # rows i = 0, 1
    x2 = np.array([0.0, 1.0], np.float32)          # rows j = 0, 1
    anchors = np.array([0, 1], np.int32)           # virtual ids: 0 = x1[i][0], 1 = x2[j][0]
    W = np.array([[1, 2, 3], [-4, 5, -6]], np.float32).reshape(-1)
    g = np.array([[0, 0, 0], [1, -1, 0.5]], np.float32).reshape(-1)
    u = Fraction(2) - 1                            # x1[0][0] - x2[1][0] = 1: idx 1, alt 0
    du = du_exact(u)
    dot = lambda r: sum(Fraction(int(W[r * O + o])) * Fraction(float(g[O + o])) for o in range(O))
    p = trunc_payload(du * (dot(1) - dot(0)), 0.5)
    xg, _, wg = oracle.propagate_product(x1, x2, None, anchors, W, g, 1, 2, n1, n2, 0, 1, 1, O,
                                         lr=0.5, int_mode=True, int_rescaler=0.5,
                                         w_grad=np.zeros(2 * O, np.float32), same_x=False)[:3]
    x2g = oracle.propagate_product(x1, x2, None, anchors, W, g, 1, 2, n1, n2, 0, 1, 1, O, lr=0.5,
                                   int_mode=True, int_rescaler=0.5, same_x=False)[3]
    assert i32(xg)[0] == p and i32(xg)[1] == 0
    assert i32(x2g)[1] == -p and i32(x2g)[0] == 0
    # (-4 - 5 - 3) - (1 - 2 + 1.5) = -12.5; du = 1/8: term -25/16, times D/2
    assert p == -(25 * DENOM // 32)
    expect = np.zeros((2, O), np.int64)
    expect[1] = [trunc_payload(Fraction(float(v)) / 2, 0.5) for v in g[O:]]
    assert np.array_equal(i32(wg).reshape(2, O).astype(np.int64), expect)
    assert expect[1, 1] == -(DENOM // 4)
