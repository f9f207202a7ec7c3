"""Pins of the product-mode oracle (concatenation_product=False): an
independent restatement that builds every pair's virtual input row the way
the reference's GTLUTProduct does (src/spiky/lut/tests/gt_lut_product.py:
137-180: concatenation [x1[i], x2[j], pe] or the sliced interleaving) and
looks it up, plus closed forms of the backward."""
import numpy as np
import pytest


def _triple(x, b, i, j, pe_t, S, n, sliced):
    a, c = x[(b * S + i) * n:(b * S + i + 1) * n], x[(b * S + j) * n:(b * S + j + 1) * n]
    if sliced:
        return np.stack([a, c, pe_t], axis=1).reshape(-1)
    return np.concatenate([a, c] + ([pe_t] if pe_t is not None else []))


def _lookup(row, anc, eps):
    idx, md, flip = 0, np.float32(3.4e38), -1
    picks = None
    for k in range(anc.shape[0]):
        a1, a2 = anc[k]
        if a1 < 0 or a2 < 0:
            continue
        d = np.float32(row[a1] - row[a2])
        if (d > 0) if eps == 0 else (abs(d) >= eps and d > 0):
            idx |= 1 << k
        if abs(d) < abs(md):
            md, flip, picks = d, k, (a1, a2)
    return idx, (idx ^ (1 << flip) if flip >= 0 else idx), md, picks


def _case(seed, sliced, pd):
    rng = np.random.default_rng(seed)
    B, S, n, T, Nc, O = 2, 6, 3 if not sliced else 4, 5, 3, 7
    if sliced:
        pd = n
    x = rng.standard_normal(B * S * n).astype(np.float32)
    pe = rng.standard_normal((S - 1) * T * pd).astype(np.float32) if pd else None
    width = 2 * n + pd if not sliced else 3 * n
    anc = rng.integers(0, width, size=(T, Nc, 2)).astype(np.int32)
    anc[1, 2] = -1  # an unused pair
    w = rng.integers(-4, 5, size=(T * (1 << Nc) * O)).astype(np.float32)
    return B, S, n, T, Nc, O, pd, x, pe, anc, w


@pytest.mark.parametrize("sliced,pd,eps", [(False, 2, 0.0), (False, 0, 0.0), (True, 0, 0.0), (False, 2, 0.3)])
def test_product_forward_matches_triple_restatement(oracle, sliced, pd, eps):
    B, S, n, T, Nc, O, pd, x, pe, anc, w = _case(3, sliced, pd)
    E = 1 << Nc
    want = np.zeros((B, S, O), np.float32)
    for b in range(B):
        for j in range(S):
            for t in range(T):
                for i in range(j):
                    pe_t = pe[((j - i - 1) * T + t) * pd:((j - i - 1) * T + t + 1) * pd] if pd else None
                    idx, _, _, _ = _lookup(_triple(x, b, i, j, pe_t, S, n, sliced), anc[t], eps)
                    want[b, j] += w[(t * E + idx) * O:(t * E + idx + 1) * O]
    got = oracle.fill_outputs_product(x, x, pe, anc.reshape(-1), w, B, S, n, n, pd, T, Nc, O,
                                      sliced=sliced, cmp_eps=eps)
    assert np.array_equal(got, want.reshape(-1))  # integer weights: exact


@pytest.mark.parametrize("sliced,pd", [(False, 2), (True, 0)])
def test_product_backward_closed_forms(oracle, sliced, pd):
    B, S, n, T, Nc, O, pd, x, pe, anc, w = _case(5, sliced, pd)
    E = 1 << Nc
    rng = np.random.default_rng(9)
    g = rng.integers(-3, 4, size=B * S * O).astype(np.float32)
    lr = 0.5
    xg, pg, wg = oracle.propagate_product(x, x, pe, anc.reshape(-1), w, g, B, S, n, n, pd, T, Nc, O,
                                          sliced=sliced, lr=lr, w_grad=np.zeros_like(w))
    # every pair pushes +du and -du: the gradient entries sum to zero
    tot = np.float64(xg.sum(dtype=np.float64)) + (np.float64(pg.sum(dtype=np.float64)) if pg is not None else 0.0)
    assert abs(tot) <= 1e-5 * (np.abs(xg).sum() + (np.abs(pg).sum() if pg is not None else 0.0) + 1e-30)
    # each (b, j, t) adds lr * g[b, j] to one row per pair i < j: column sums are closed form
    gs = g.reshape(B, S, O)
    col = lr * sum(j * gs[b, j] for b in range(B) for j in range(S))
    per_table = wg.reshape(T, E, O).sum(axis=1, dtype=np.float64)
    for t in range(T):
        assert np.array_equal(per_table[t], col.astype(np.float64))
    # du of one pair by hand: the first pair (b=0, j=1, i=0, t=0) alone
    g1 = np.zeros_like(g)
    g1[(0 * S + 1) * O:(0 * S + 2) * O] = g[(0 * S + 1) * O:(0 * S + 2) * O]
    xg1, pg1, _ = oracle.propagate_product(x, x, pe, anc[:1].reshape(-1), w[:E * O], g1, B, S, n, n,
                                           pd, 1, Nc, O, sliced=sliced)
    pe_t = pe[0:pd] if pd else None
    row = _triple(x, 0, 0, 1, pe_t, S, n, sliced)
    idx, alt, md, (a1, a2) = _lookup(row, anc[0], 0.0)
    gj = g1[(0 * S + 1) * O:(0 * S + 2) * O].astype(np.float64)
    dm = (w[idx * O:(idx + 1) * O].astype(np.float64) @ gj) - (w[alt * O:(alt + 1) * O].astype(np.float64) @ gj)
    u = np.float64(md)
    r = 1.0 / (1.0 + abs(u))
    du = (0.5 * r * r if u > 0 else -0.5 * r * r) * dm
    full = np.concatenate([xg1, pg1 if pg1 is not None else np.zeros(0, np.float32)])
    nz = np.flatnonzero(full)
    if abs(du) > 1e-17 and a1 != a2:
        assert sorted(np.round(full[nz], 5).tolist()) == sorted(np.round([np.float32(du), np.float32(-du)], 5).tolist())


@pytest.mark.parametrize("sliced,pd", [(False, 2), (True, 0)])
def test_product_fp64_mode_walks_the_same_terms(oracle, sliced, pd):
    """The fp64 tolerance mode must visit exactly the terms of the serial
    oracle: with integer weights and gradients every sum is exact in both, so
    they agree bit for bit, and abs bounds |sum|."""
    B, S, n, T, Nc, O, pd, x, pe, anc, w = _case(11, sliced, pd)
    rng = np.random.default_rng(5)
    g = rng.integers(-3, 4, size=B * S * O).astype(np.float32)
    a = anc.reshape(-1)
    out = oracle.fill_outputs_product(x, x, pe, a, w, B, S, n, n, pd, T, Nc, O, sliced=sliced)
    tot, mag = oracle.fill_outputs_product64(x, x, pe, a, w, B, S, n, n, pd, T, Nc, O, sliced=sliced)
    assert np.array_equal(tot, out.astype(np.float64))
    assert np.all(mag >= np.abs(tot)) and mag.max() > 0
    wg = np.zeros(w.size, np.float32)
    xg, peg, wg = oracle.propagate_product(x, x, pe, a, w, g, B, S, n, n, pd, T, Nc, O, sliced=sliced,
                                           lr=1.0, w_grad=wg)
    r = oracle.propagate_product64(x, x, pe, a, w, g, B, S, n, n, pd, T, Nc, O, sliced=sliced, lr=1.0)
    assert np.array_equal(r["w"][0], wg.astype(np.float64))
    # du terms are not integers: the fp32 serial sums lie within the bound
    n_terms = 2 * T * S
    assert np.all(np.abs(xg - r["x"][0]) <= n_terms * 2.0 ** -24 * r["x"][1])
    if pd:
        assert np.all(np.abs(peg - r["pe"][0]) <= n_terms * 2.0 ** -24 * r["pe"][1])
    assert r["x"][1].max() > 0


def _full_csr(T, E, O):
    n = T * E
    return np.arange(n + 1, dtype=np.int64) * O, np.tile(np.arange(O, dtype=np.int32), n)


@pytest.mark.parametrize("sliced,pd", [(False, 2), (True, 0)])
def test_product_sparse_full_connectivity_is_the_fc_path(oracle, sliced, pd):
    """A CSR that lists every output of every neuron in order turns the sparse
    product functions into the FC ones: equal outputs, input, positional and
    weight gradients (int32 payloads bit for bit; integer fp32 values exactly)."""
    B, S, n, T, Nc, O, pd, x, pe, anc, w = _case(31, sliced, pd)
    a = anc.reshape(-1)
    off, tg = _full_csr(T, 1 << Nc, O)
    geo = (B, S, n, n, pd, T, Nc, O)
    assert np.array_equal(oracle.fill_outputs_product(x, x, pe, a, w, *geo, sliced=sliced),
                          oracle.fill_outputs_product_sparse(x, x, pe, a, w, off, tg, *geo, sliced=sliced))
    rng = np.random.default_rng(6)
    g = rng.standard_normal(B * S * O).astype(np.float32)
    fc = oracle.propagate_product(x, x, pe, a, w, g, *geo, sliced=sliced, lr=0.5, int_mode=True,
                                  int_rescaler=0.01, w_grad=np.zeros(w.size, np.float32))
    sp = oracle.propagate_product_sparse(x, x, pe, a, w, off, tg, g, *geo, sliced=sliced, lr=0.5,
                                         int_mode=True, int_rescaler=0.01)
    for u, v in zip(fc, sp):
        if u is not None:
            assert np.array_equal(u.view(np.int32), v.view(np.int32))
    f64 = oracle.propagate_product64(x, x, pe, a, w, g, *geo, sliced=sliced, lr=0.5)
    s64 = oracle.propagate_product_sparse(x, x, pe, a, w, off, tg, g, *geo, sliced=sliced, lr=0.5, bounds=True)
    for k in ("x", "pe", "w"):
        if f64[k] is not None:
            assert np.array_equal(f64[k][0], s64[k][0]) and np.array_equal(f64[k][1], s64[k][1])


def test_product_sparse_brute_force(oracle):
    """A random ragged topology (empty neurons, repeated targets) against a
    direct loop over pairs and synapses, integer weights (exact)."""
    B, S, n, T, Nc, O, pd, x, pe, anc, _ = _case(32, False, 2)
    rng = np.random.default_rng(7)
    E = 1 << Nc
    counts = rng.integers(0, 6, size=T * E)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    tg = rng.integers(0, O, size=off[-1]).astype(np.int32)
    w = rng.integers(-4, 5, size=off[-1]).astype(np.float32)
    got = oracle.fill_outputs_product_sparse(x, x, pe, anc.reshape(-1), w, off, tg, B, S, n, n, pd, T, Nc, O)
    want = np.zeros((B, S, O))
    for b in range(B):
        for j in range(S):
            for t in range(T):
                for i in range(j):
                    pe_t = pe[((j - i - 1) * T + t) * pd:((j - i - 1) * T + t + 1) * pd]
                    idx, _, _, _ = _lookup(_triple(x, b, i, j, pe_t, S, n, False), anc[t], 0.0)
                    m = t * E + idx
                    for s_ in range(off[m], off[m + 1]):
                        want[b, j, tg[s_]] += w[s_]
    assert np.array_equal(got, want.reshape(-1).astype(np.float32))
