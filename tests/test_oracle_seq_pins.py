"""Pins the sequence-concat functions of the CPU oracle against an independent
numpy restatement of the reference's ground-truth attention head
(src/spiky/lut/tests/gt_lut_transformer.py:268-426: every causal pair
pos1 < pos looks up row Q_pos | K_pos1 | PE_(pos-pos1-1); the backward flips
Q's min anchor if |dQ| < |dK| else K's, and PE's when |dPE| is strictly the
smallest), plus rounding-point and special-case checks a plausible mistake
(swapped Q/K, wrong PE offset, fp32 instead of fp64 pair sums, an EPS cut on
the positional gradient) fails.
"""
import numpy as np
import pytest


def up(u):
    """gt_lut_transformer.py:28-30 (sign(0) = -1)."""
    s = 1.0 if u > 0 else -1.0
    return 0.5 * s / (1 + abs(u)) / (1 + abs(u))


def rand_case(rng, B, S, I, T, Nc, Npe, O, int_weights=False):
    E = 1 << (2 * Nc + Npe)
    idx = rng.integers(0, 1 << Nc, size=(B, S, T)).astype(np.int32)
    md = rng.standard_normal((B, S, T)).astype(np.float32)
    mi = rng.integers(0, Nc, size=(B, S, T)).astype(np.int32)
    pidx = rng.integers(0, 1 << max(Npe, 1), size=(S - 1, T)).astype(np.int32) if Npe else None
    pmd = rng.uniform(-1, 1, size=(S - 1, T)).astype(np.float32) if Npe else None
    pmi = rng.integers(0, Npe, size=(S - 1, T)).astype(np.int32) if Npe else None
    if int_weights:
        W = rng.integers(-8, 9, size=T * E * O).astype(np.float32)
    else:
        W = (rng.standard_normal(T * E * O) * 0.01).astype(np.float32)
    anchors = np.stack([rng.choice(I, 2, replace=False) for _ in range(T * Nc)]).astype(np.int32).reshape(-1)
    return idx, md, mi, pidx, pmd, pmi, W, anchors


def np_row(q, k, p, Nc, Npe):
    return (q << (Nc + Npe)) | (k << Npe) | p


def np_seq_forward(W, idx, pidx, B, S, T, Nc, Npe, O):
    E = 1 << (2 * Nc + Npe)
    Wr = W.reshape(T, E, O).astype(np.float64)
    out = np.zeros((B, S, O), np.float64)
    for b in range(B):
        for t in range(T):
            for pos1 in range(S):
                for pos in range(pos1 + 1, S):
                    p = pidx[pos - pos1 - 1, t] if Npe else 0
                    out[b, pos] += Wr[t, np_row(idx[b, pos, t], idx[b, pos1, t], p, Nc, Npe)]
    return out


def np_seq_backward(W, g, idx, md, mi, pidx, pmd, pmi, anchors, B, S, I, T, Nc, Npe, O):
    """One block of outputs (O <= ogs): the textbook head backward in fp64."""
    E = 1 << (2 * Nc + Npe)
    Wr = W.reshape(T, E, O).astype(np.float64)
    ap = anchors.reshape(T, Nc, 2)
    xg = np.zeros((B, S, I), np.float64)
    peg = np.zeros((max(S - 1, 1), T, max(Npe, 1)), np.float64)
    wg = np.zeros((T, E, O), np.float64)
    for b in range(B):
        for pos in range(1, S):
            gy = g[b, pos].astype(np.float64)
            for pos1 in range(pos):
                d = pos - pos1 - 1
                for t in range(T):
                    Q, K = idx[b, pos, t], idx[b, pos1, t]
                    P = pidx[d, t] if Npe else 0
                    r = np_row(Q, K, P, Nc, Npe)
                    if abs(md[b, pos, t]) < abs(md[b, pos1, t]):
                        m = mi[b, pos, t]
                        rb = np_row(Q ^ (1 << m), K, P, Nc, Npe)
                        delta = gy @ (Wr[t, r] - Wr[t, rb]) * up(np.float64(md[b, pos, t]))
                        xg[b, pos, ap[t, m, 0]] += delta
                        xg[b, pos, ap[t, m, 1]] -= delta
                    else:
                        m = mi[b, pos1, t]
                        rb = np_row(Q, K ^ (1 << m), P, Nc, Npe)
                        delta = gy @ (Wr[t, r] - Wr[t, rb]) * up(np.float64(md[b, pos1, t]))
                        xg[b, pos1, ap[t, m, 0]] += delta
                        xg[b, pos1, ap[t, m, 1]] -= delta
                    if Npe and abs(pmd[d, t]) < abs(md[b, pos, t]) and abs(pmd[d, t]) < abs(md[b, pos1, t]):
                        rp = np_row(Q, K, P ^ (1 << pmi[d, t]), Nc, Npe)
                        peg[d, t, pmi[d, t]] += gy @ (Wr[t, r] - Wr[t, rp]) * up(np.float64(pmd[d, t]))
                    wg[t, r] += gy
    return xg, peg, wg


@pytest.mark.parametrize("Npe", [0, 3])
def test_seq_forward_exact_integer_tables(oracle, Npe):
    rng = np.random.default_rng(1)
    B, S, I, T, Nc, O = 2, 7, 10, 3, 2, 5
    idx, md, mi, pidx, pmd, pmi, W, anchors = rand_case(rng, B, S, I, T, Nc, Npe, O, int_weights=True)
    out = oracle.fill_outputs_seq(W, idx, pidx, B, O, T, S, Nc, Npe)
    ref = np_seq_forward(W, idx, pidx, B, S, T, Nc, Npe, O)
    assert np.array_equal(out.reshape(B, S, O), ref.astype(np.float32))
    assert np.all(out.reshape(B, S, O)[:, 0] == 0)  # position 0 has no earlier token


def test_seq_forward_fp64_pair_sum(oracle):
    """The pairs of one (b, j, t) are summed in fp64 and committed once:
    1e8 + 1 - 1e8 gives 1 (an fp32 running sum would give 0)."""
    B, S, T, Nc, Npe, O = 1, 4, 1, 1, 0, 1
    E = 1 << (2 * Nc)
    idx = np.array([[[0]], [[1]], [[0]], [[0]]], np.int32).reshape(B, S, T)
    W = np.zeros(T * E * O, np.float32)
    # j = 3: pairs i = 0, 1, 2 -> rows (Q=0,K=0), (0,1), (0,0)
    W[np_row(0, 0, 0, Nc, Npe)] = 1e8
    W[np_row(0, 1, 0, Nc, Npe)] = 1.0
    out = oracle.fill_outputs_seq(W, idx, None, B, O, T, S, Nc, Npe)
    assert out[3] == np.float32(2e8 + 1)
    W[np_row(0, 0, 0, Nc, Npe)] = 0.0
    W[np_row(0, 1, 0, Nc, Npe)] = 1.0
    W[np_row(1, 0, 0, Nc, Npe)] = 1e8
    W[np_row(0, 0, 0, Nc, Npe)] = -1e8
    out = oracle.fill_outputs_seq(W, idx, None, B, O, T, S, Nc, Npe)
    # j = 3 (Q=0): rows (0,0)=-1e8, (0,1)=1, (0,0)=-1e8 -> -2e8 + 1 exactly in fp64
    assert out[3] == np.float32(-2e8 + 1)
    # j = 1 (Q=1): one pair (1, 0) = 1e8
    assert out[1] == np.float32(1e8)


@pytest.mark.parametrize("Npe", [0, 2])
def test_seq_backward_matches_ground_truth(oracle, Npe):
    rng = np.random.default_rng(2 + Npe)
    B, S, I, T, Nc, O = 2, 9, 12, 3, 3, 6
    idx, md, mi, pidx, pmd, pmi, W, anchors = rand_case(rng, B, S, I, T, Nc, Npe, O)
    g = rng.standard_normal((B, S, O)).astype(np.float32)
    xg, peg = oracle.propagate_seq(W, g, idx, md, mi, pidx, pmd, pmi, anchors, B, I, O, T, S, Nc,
                                   Npe, ogs=32)
    rxg, rpeg, rwg = np_seq_backward(W, g, idx, md, mi, pidx, pmd, pmi, anchors, B, S, I, T, Nc,
                                     Npe, O)
    scale = np.abs(rxg).max()
    assert np.abs(xg.reshape(B, S, I) - rxg).max() <= 1e-6 * scale
    if Npe:
        assert np.abs(peg.reshape(S - 1, T, Npe) - rpeg).max() <= 1e-6 * np.abs(rpeg).max()
        assert np.count_nonzero(rpeg) > 0
    # integer-valued gradients make every fp32 sum exact: the weight gradient is np.add.at
    gi = rng.integers(-4, 5, size=(B, S, O)).astype(np.float32)
    wg = np.zeros(W.size, np.float32)
    oracle.gather_wgrad_seq(gi, idx, pidx, wg, B, O, T, S, Nc, Npe, ogs=4)
    _, _, rwg = np_seq_backward(W, gi, idx, md, mi, pidx, pmd, pmi, anchors, B, S, I, T, Nc, Npe, O)
    assert np.array_equal(wg, rwg.reshape(-1).astype(np.float32))


def test_seq_positional_gradient_has_no_eps_cut(oracle):
    """update_positional_gradients (proto:1016-1046) commits every term, while
    the input gradient drops |du| <= 1e-17 (proto:833)."""
    B, S, I, T, Nc, Npe, O = 1, 2, 4, 1, 1, 1, 1
    E = 1 << (2 * Nc + Npe)
    idx = np.zeros((B, S, T), np.int32)
    md = np.full((B, S, T), 0.5, np.float32)
    mi = np.zeros((B, S, T), np.int32)
    pidx = np.zeros((S - 1, T), np.int32)
    pmd = np.full((S - 1, T), 0.1, np.float32)
    pmi = np.zeros((S - 1, T), np.int32)
    anchors = np.array([0, 1], np.int32)
    W = np.zeros(T * E * O, np.float32)
    W[np_row(0, 0, 1, Nc, Npe)] = -1e-20      # PE-flipped row
    g = np.ones((B, S, O), np.float32)
    xg, peg = oracle.propagate_seq(W, g, idx, md, mi, pidx, pmd, pmi, anchors, B, I, O, T, S, Nc, Npe)
    assert np.all(xg == 0)
    assert peg[0] == np.float32(up(np.float64(np.float32(0.1))) * 1e-20)


def test_check_pe_special_cases(oracle):
    pe = np.array([0.0, -0.25, 0.25, 0.5,    # ties on |v| -> first; 0 -> bit 0
                   -0.1, 0.3, -0.3, 0.05], np.float32)
    pidx, pmd, pmi = oracle.check_pe(pe, 3, 1, 4)
    assert list(pidx) == [0b1100, 0b1010]
    assert list(pmi) == [0, 3] and list(pmd) == [np.float32(0.0), np.float32(0.05)]
    pidx = oracle.check_pe(pe, 3, 1, 4, cmp_eps=0.3, train=False)
    # |v| < eps -> bit 0; |v| == eps is outside the band (misc.h:16)
    assert list(pidx) == [0b1000, 0b0010]


def test_seq_backward_fp64_accumulation(oracle):
    """acc64 sums the same terms as the fp32 restatement: equal after rounding
    when every element gets one term (S = 2, one block), and within the fp32
    summation bound n * 2^-24 * sum|partial| otherwise."""
    rng = np.random.default_rng(21)
    for B, S, I, T, Nc, Npe, O in ((3, 2, 40, 1, 3, 2, 16), (2, 24, 12, 5, 3, 2, 40)):
        x = rng.standard_normal(B * S * I).astype(np.float32)
        anchors = np.concatenate([rng.permutation(I)[:2] for _ in range(T * Nc)]).astype(np.int32)
        W = (rng.standard_normal(T * (1 << (2 * Nc + Npe)) * O) * 0.01).astype(np.float32)
        pe = rng.uniform(-1, 1, (S - 1) * T * Npe).astype(np.float32)
        g = rng.standard_normal(B * S * O).astype(np.float32)
        idx, md, mi = oracle.check_detectors(x, anchors, B * S, I, T, Nc)
        pli, pmd, pmi = oracle.check_pe(pe, S, T, Npe)
        args = (W, g, idx, md, mi, pli, pmd, pmi, anchors, B, I, O, T, S, Nc, Npe)
        xg32, pg32 = oracle.propagate_seq(*args)
        xg64, pg64 = oracle.propagate_seq(*args, acc64=True)
        assert xg64.dtype == np.float64
        if S == 2:
            # anchors are distinct per table and T = 1: one term per element
            assert np.array_equal(xg64.astype(np.float32), xg32)
            assert np.array_equal(pg64.astype(np.float32), pg32)
        else:
            n = S * T * ((O + 31) // 32)
            scale = np.abs(xg64).reshape(B * S, I).max(axis=1, keepdims=True) * 4 + 1e-30
            err = np.abs(xg32.astype(np.float64) - xg64).reshape(B * S, I)
            assert np.all(err <= n * 2.0 ** -24 * scale)


# ---------------------------------------------------------------- sparse connectivity
def full_csr(T, E, O):
    """Every lookup neuron targets every output in order: the sparse layout of
    an FC table (synapse n*O + o is W[n][o])."""
    n = T * E
    return (np.arange(n + 1, dtype=np.int64) * O, np.tile(np.arange(O, dtype=np.int32), n))


@pytest.mark.parametrize("Npe", [0, 2])
def test_seq_sparse_full_connectivity_is_the_fc_path(oracle, Npe):
    """With a CSR that lists every output of every neuron in order and groups
    of ogs synapses, the sparse sequence functions see exactly the FC terms:
    forward and weight gradient equal the FC oracle (integer values, exact);
    int32 input / positional gradients equal bit for bit; fp32 ones hold the
    same terms (both within their fp32 bound of the fp64 sum)."""
    rng = np.random.default_rng(21)
    B, S, I, T, Nc, O, ogs = 2, 7, 9, 3, 2, 10, 4
    E = 1 << (2 * Nc + Npe)
    idx, md, mi, pidx, pmd, pmi, W, anchors = rand_case(rng, B, S, I, T, Nc, Npe, O, int_weights=True)
    off, tg = full_csr(T, E, O)
    n_grp = (O + ogs - 1) // ogs
    f_fc = oracle.fill_outputs_seq(W, idx.reshape(-1), pidx, B, O, T, S, Nc, Npe)
    f_sp = oracle.fill_outputs_seq_sparse(W, idx.reshape(-1), pidx, off, tg, B, S, O, T, Nc, Npe, ogs, n_grp)
    assert np.array_equal(f_fc, f_sp)
    gi = rng.integers(-3, 4, size=B * S * O).astype(np.float32)
    w_fc = np.zeros(W.size, np.float32)
    oracle.gather_wgrad_seq(gi, idx.reshape(-1), pidx, w_fc, B, O, T, S, Nc, Npe, ogs=ogs, first_meta_lr=0.5)
    w_sp = oracle.gather_wgrad_seq_sparse(gi, idx.reshape(-1), pidx, off, tg, B, S, O, T, Nc, Npe, ogs, n_grp,
                                          lr=0.5)
    assert np.array_equal(w_fc, w_sp)
    g = rng.standard_normal(B * S * O).astype(np.float32)
    args = (W, g, idx.reshape(-1), md.reshape(-1), mi.reshape(-1), pidx, pmd, pmi, anchors)
    xi_fc, pi_fc = oracle.propagate_seq(*args, B, I, O, T, S, Nc, Npe, ogs=ogs, int_mode=True, int_rescaler=0.01)
    xi_sp, pi_sp = oracle.propagate_seq_sparse(*args, off, tg, B, I, O, T, S, Nc, Npe, ogs, n_grp,
                                               int_mode=True, int_rescaler=0.01)
    assert np.array_equal(xi_fc.view(np.int32), xi_sp.view(np.int32))
    if Npe:
        assert np.array_equal(pi_fc.view(np.int32), pi_sp.view(np.int32))
    xf, pf, (xs, xa), pb = oracle.propagate_seq_sparse(*args, off, tg, B, I, O, T, S, Nc, Npe, ogs, n_grp,
                                                       bounds=True)
    x64, _ = oracle.propagate_seq(*args, B, I, O, T, S, Nc, Npe, ogs=ogs, acc64=True)
    n = 2 * T * S * n_grp
    assert np.all(np.abs(x64 - xs) <= n * 2.0 ** -24 * xa + 1e-30)  # same terms
    assert np.all(np.abs(xf - xs) <= n * 2.0 ** -24 * xa)
    assert xa.max() > 0


def test_seq_sparse_forward_brute_force(oracle):
    """A random sparse topology (ragged neurons, empty ones, repeated targets)
    against a direct loop over pairs and synapses, integer weights (exact)."""
    rng = np.random.default_rng(22)
    B, S, T, Nc, Npe, O, fgs = 2, 6, 2, 2, 1, 7, 3
    E = 1 << (2 * Nc + Npe)
    counts = rng.integers(0, 8, size=T * E)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    tg = rng.integers(0, O, size=off[-1]).astype(np.int32)
    W = rng.integers(-5, 6, size=off[-1]).astype(np.float32)
    idx = rng.integers(0, 1 << Nc, size=(B, S, T)).astype(np.int32)
    pidx = rng.integers(0, 1 << Npe, size=(S - 1, T)).astype(np.int32)
    max_groups = int((counts.max() + fgs - 1) // fgs)
    got = oracle.fill_outputs_seq_sparse(W, idx.reshape(-1), pidx, off, tg, B, S, O, T, Nc, Npe, fgs, max_groups)
    want = np.zeros((B, S, O), np.float64)
    for b in range(B):
        for j in range(S):
            for i in range(j):
                for t in range(T):
                    n = t * E + np_row(idx[b, j, t], idx[b, i, t], pidx[j - i - 1, t], Nc, Npe)
                    for s_ in range(off[n], off[n + 1]):
                        want[b, j, tg[s_]] += W[s_]
    assert np.array_equal(got, want.reshape(-1).astype(np.float32))
