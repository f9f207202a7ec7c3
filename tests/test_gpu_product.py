"""GPU parity of product mode (concatenation_product=False; spiky_amd/csrc/
lut_product.hip behind spiky_lut_forward_step_product /
spiky_lut_backward_backprop_product) against the CPU oracle
(oracle/lut_oracle.c, restating lut_runtime_kernels_logic.proto:32-181,
2148-2264, 2396-2628).

Bars:
  * int32 summation: every accumulator bit-exact (wrapping int32 sums of the
    reference's payloads do not depend on order);
  * fp32 forward: the fp64 sum of the reference's terms rounded once,
    |gpu - s| <= 2^-24 |s| + 2^-40 a, where (s, a) are the oracle's fp64 sum
    and magnitude sum of those terms (oracle.fill_outputs_product64);
  * fp32 input, positional and weight gradients: the GPU sums the same terms
    in an order of its own, so |gpu - s| <= (n + 2) 2^-24 a + n 1e-17, n the
    most terms one element can receive -- the bound that holds for any fp32
    summation order, the reference's serial one included (pinned in
    tests/test_oracle_product_pins.py), plus the sub-EPS pushes (< 1e-17) the
    cut may keep or drop on either side.
"""
import numpy as np
import pytest
import torch

from spiky_amd import LUTDataManagerF, LUTDataManagerI

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def within(gpu, s, a, n, what):
    gpu = np.asarray(gpu, dtype=np.float64)
    bound = (n + 2) * U * a + n * 1e-17
    err = np.abs(gpu - s)
    assert np.all(err <= bound), f"{what}: max excess {np.max(err - bound)} at {np.argmax(err - bound)}"


def product_inputs(seed, B, S, n, T, Nc, O, pd, sliced):
    rng = np.random.default_rng(seed)
    width = 3 * n if sliced else 2 * n + pd
    x = rng.standard_normal(B * S * n).astype(np.float32)
    pe = rng.uniform(-1, 1, (S - 1) * T * pd).astype(np.float32) if pd else None
    anc = np.stack([rng.choice(width, 2, replace=False) for _ in range(T * Nc)]).astype(np.int32)
    anc[rng.random(T * Nc) < 0.1] = -1  # unused pairs
    W = (rng.standard_normal(T * (1 << Nc) * O) * 0.1).astype(np.float32)
    g = rng.standard_normal(B * S * O).astype(np.float32)
    return x, pe, anc.reshape(-1), W, g


def make_dm(n, O, T, Nc, pd, int_rescaler=None, lr=1.0):
    args = (2 * n + pd, O, T, Nc, 1, pd, 0, 32, 32)
    dm = LUTDataManagerF(*args) if int_rescaler is None else LUTDataManagerI(*args, int_rescaler)
    dm.register_synapse_meta(lr, -10.0, 10.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    return dm


def run_product(oracle, B, S, n, T, Nc, O, pd, sliced=False, int_rescaler=None, internal=False,
                eps=0.0, seed=0, lr=1.0, ext_lr=0.1):
    dev = torch.device("cuda:0")
    if sliced:
        pd = n
    int_mode = int_rescaler is not None
    print(f"[product] B={B} S={S} n={n} T={T} Nc={Nc} O={O} pd={pd} sliced={sliced} int={int_mode} "
          f"internal={internal} eps={eps}", flush=True)
    x, pe, anc, W, g = product_inputs(seed, B, S, n, T, Nc, O, pd, sliced)
    dm = make_dm(n, O, T, Nc, pd, int_rescaler, lr)
    xd, ad, Wd, gd = (torch.from_numpy(v).to(dev) for v in (x, anc, W, g))
    ped = torch.from_numpy(pe).to(dev) if pd else None
    out = torch.zeros(B * S * O, device=dev)
    dm.forward_step_product(Wd, B, S, xd, xd, ad, out, n, n, sliced, eps, ped)
    xg = torch.zeros(B * S * n, device=dev)
    peg = torch.zeros((S - 1) * T * pd, device=dev) if pd else None
    W_before = W.copy()
    wg = None
    if internal:
        dm.backward_backprop_product(Wd, B, S, xd, xd, ad, gd, xg, xg, ext_lr, n, n, sliced, eps, None,
                                     ped, peg)
    else:
        wg = torch.zeros_like(Wd)
        dm.backward_backprop_product(Wd, B, S, xd, xd, ad, gd, xg, xg, -1.0, n, n, sliced, eps, wg, ped,
                                     peg)
    torch.cuda.synchronize()
    got = {"out": out.cpu().numpy(), "x": xg.cpu().numpy(), "pe": peg.cpu().numpy() if pd else None,
           "w": wg.cpu().numpy() if wg is not None else None, "W": Wd.cpu().numpy()}
    geo = (B, S, n, n, pd, T, Nc, O)
    eff_lr = lr * (-ext_lr if internal else 1.0)
    if int_mode:
        rout = oracle.fill_outputs_product(x, x, pe, anc, W, *geo, sliced=sliced, cmp_eps=eps,
                                           int_mode=True, int_rescaler=int_rescaler)
        rwg = np.zeros(W.size, np.float32)
        rxg, rpeg, rwg = oracle.propagate_product(x, x, pe, anc, W, g, *geo, sliced=sliced, cmp_eps=eps,
                                                  lr=eff_lr, int_mode=True, int_rescaler=int_rescaler,
                                                  w_grad=rwg)
        for buf in (rout, rxg, rpeg, rwg):
            if buf is not None:
                oracle.convert_int_to_float(buf, int_rescaler)
        assert np.array_equal(got["out"], rout)
        assert np.array_equal(got["x"], rxg)
        if pd:
            assert np.array_equal(got["pe"], rpeg)
        assert np.array_equal(got["w"], rwg)
        return got
    s, a = oracle.fill_outputs_product64(x, x, pe, anc, W, *geo, sliced=sliced, cmp_eps=eps)
    err = np.abs(got["out"].astype(np.float64) - s)
    assert np.all(err <= U * np.abs(s) + 2.0 ** -40 * a), f"forward: max err {err.max()}"
    r = oracle.propagate_product64(x, x, pe, anc, W, g, *geo, sliced=sliced, cmp_eps=eps, lr=eff_lr)
    within(got["x"], *r["x"], 2 * T * S, "x_grad")
    if pd:
        within(got["pe"], *r["pe"], 2 * B * S, "pe_grad")
    n_w = B * S * (S - 1) // 2
    if internal:
        # W += sum of the terms (lut_runtime.cu:1130-1160), after du used the old W
        within(got["W"], W_before.astype(np.float64) + r["w"][0], r["w"][1] + np.abs(W_before), n_w,
               "weights (Internal)")
    else:
        within(got["w"], *r["w"], n_w, "w_grad")
        assert np.array_equal(got["W"], W_before)
    assert np.abs(got["x"]).max() > 0
    return got


@pytest.mark.parametrize("pd", [0, 3])
def test_product_fp32(oracle, cuda_device, pd):
    run_product(oracle, B=3, S=12, n=10, T=6, Nc=4, O=40, pd=pd, seed=1)


def test_product_sliced(oracle, cuda_device):
    run_product(oracle, B=2, S=9, n=8, T=5, Nc=5, O=33, pd=0, sliced=True, seed=2)


def test_product_cmp_eps(oracle, cuda_device):
    run_product(oracle, B=2, S=8, n=6, T=4, Nc=4, O=20, pd=2, eps=0.25, seed=3)


@pytest.mark.parametrize("sliced", [False, True])
def test_product_int32_bit_exact(oracle, cuda_device, sliced):
    run_product(oracle, B=3, S=10, n=8, T=6, Nc=4, O=36, pd=2, sliced=sliced, int_rescaler=0.001,
                seed=4)


def test_product_internal_policy(oracle, cuda_device):
    run_product(oracle, B=2, S=10, n=8, T=4, Nc=4, O=24, pd=2, internal=True, lr=0.5, ext_lr=0.2,
                seed=5)


def test_product_wide_tables_and_tile_edges(oracle, cuda_device):
    """256-row tables, and T*E, B*S and O that are not multiples of the
    64-wide product tiles."""
    run_product(oracle, B=3, S=23, n=16, T=5, Nc=8, O=70, pd=4, seed=6)


def test_product_largest_histogram_int32(oracle, cuda_device):
    """T * 2^n_anchors = 16384, the largest per-(b, j) count table."""
    run_product(oracle, B=1, S=5, n=12, T=64, Nc=8, O=8, pd=0, int_rescaler=0.01, seed=7)


def test_product_long_sequence_global_path(oracle, cuda_device):
    """A sequence too long for the table-major pass (its 2*Nc anchor inputs of
    every position, S * 12 * 4 bytes, beyond the 64 KB LDS budget) takes the
    pass that reads the rows from global memory."""
    run_product(oracle, B=1, S=1400, n=8, T=3, Nc=6, O=8, pd=2, seed=10)
    run_product(oracle, B=1, S=1400, n=8, T=3, Nc=6, O=8, pd=2, int_rescaler=0.001, seed=10)


def test_product_wide_rows(oracle, cuda_device):
    """Rows of 6200 inputs: only the anchor inputs are staged."""
    run_product(oracle, B=1, S=4, n=6200, T=3, Nc=3, O=8, pd=2, seed=10)


@pytest.mark.parametrize("int_rescaler", [None, 0.001])
def test_product_many_anchors(oracle, cuda_device, int_rescaler):
    """10 anchors (1024-row tables): the widest anchor bucket of the pass."""
    run_product(oracle, B=2, S=7, n=12, T=2, Nc=10, O=8, pd=3, int_rescaler=int_rescaler, seed=12)


def test_product_shortest_sequence(oracle, cuda_device):
    """S = 2: one pair per sequence; position 0 receives nothing."""
    got = run_product(oracle, B=4, S=2, n=6, T=3, Nc=3, O=10, pd=2, seed=8)
    assert np.all(got["out"].reshape(4, 2, 10)[:, 0] == 0)


def test_product_out_of_range_anchor_is_skipped(oracle, cuda_device):
    """An anchor id beyond the virtual row never reads memory: it is skipped
    like an unused (-1) pair."""
    dev = torch.device("cuda:0")
    B, S, n, T, Nc, O, pd = 2, 6, 5, 3, 3, 8, 0
    x, pe, anc, W, g = product_inputs(9, B, S, n, T, Nc, O, pd, False)
    bad = anc.copy()
    bad[0:2] = [2 * n + 1000, 1]
    skipped = anc.copy()
    skipped[0:2] = -1
    outs = []
    for a in (bad, skipped):
        dm = make_dm(n, O, T, Nc, pd)
        out = torch.zeros(B * S * O, device=dev)
        xd = torch.from_numpy(x).to(dev)
        dm.forward_step_product(torch.from_numpy(W).to(dev), B, S, xd, xd, torch.from_numpy(a).to(dev),
                                out, n, n, False, 0.0, None)
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])


# ---------------------------------------------------------------- layers
def _layer(dev, n, S, T, Nc, O, pd, sliced=False, unified=False, policy=None, summation=torch.float32,
           seed=3):
    from spiky_amd import LUTLayer
    from spiky_amd.lut.LUTLayer import GradientPolicy, GradientType
    layer = LUTLayer(n, Nc, T, O, sequence_length=S, concatenation_product=False,
                     sliced_product_mode=sliced, positional_dim=pd, unified_pe=unified,
                     weights_gradient_policy=policy or GradientPolicy(GradientType.Dense),
                     summation_dtype=summation, random_seed=seed, device=dev)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        layer._weights.copy_((torch.randn(layer._weights.numel(), generator=g) * 0.1).to(dev))
    return layer


def _full_pe(layer):
    if layer._positional_dim == 0:
        return None
    return layer._prepare_positional_embeddings().detach().cpu().numpy()


@pytest.mark.parametrize("sliced,unified,pd", [(False, False, 4), (False, True, 4), (True, False, 12),
                                               (False, False, 0)])
def test_layer_product_autograd(oracle, cuda_device, sliced, unified, pd):
    dev = cuda_device
    B, S, n, T, Nc, O = 3, 10, 12, 8, 4, 24
    print(f"[product layer] sliced={sliced} unified={unified} pd={pd}", flush=True)
    layer = _layer(dev, n, S, T, Nc, O, pd, sliced, unified)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, S, n, generator=g).to(dev).requires_grad_(True)
    y = layer(x)
    go = torch.randn(B, S, O, generator=g).to(dev)
    y.backward(go)
    torch.cuda.synchronize()
    xn = x.detach().cpu().numpy().reshape(-1)
    anc = layer._detector_anchors.cpu().numpy()
    W = layer._weights.detach().cpu().numpy()
    pe = _full_pe(layer)
    geo = (B, S, n, n, pd, T, Nc, O)
    s, a = oracle.fill_outputs_product64(xn, xn, pe, anc, W, *geo, sliced=sliced)
    yn = y.detach().cpu().numpy().reshape(-1).astype(np.float64)
    assert np.all(np.abs(yn - s) <= U * np.abs(s) + 2.0 ** -40 * a)
    r = oracle.propagate_product64(xn, xn, pe, anc, W, go.cpu().numpy().reshape(-1), *geo, sliced=sliced)
    within(x.grad.cpu().numpy().reshape(-1), *r["x"], 2 * T * S, "x.grad")
    within(layer._weights.grad.cpu().numpy(), *r["w"], B * S * (S - 1) // 2, "weights.grad")
    if pd:
        pg = layer._positional_embeddings.grad.cpu().numpy()
        ps, pa = r["pe"]
        if unified:  # the repeat over detectors sums their gradients
            ps = ps.reshape(S - 1, T, pd).sum(axis=1).reshape(-1)
            pa = pa.reshape(S - 1, T, pd).sum(axis=1).reshape(-1)
        within(pg, ps, pa, 2 * B * S * (T if unified else 1), "pe.grad")


def test_layer_product_int32_bit_exact(oracle, cuda_device):
    dev = cuda_device
    B, S, n, T, Nc, O, pd = 2, 8, 10, 6, 4, 20, 3
    layer = _layer(dev, n, S, T, Nc, O, pd, summation=torch.int32)
    R = layer._lut_dm._int_rescaler
    g = torch.Generator().manual_seed(2)
    x = torch.randn(B, S, n, generator=g).to(dev).requires_grad_(True)
    y = layer(x)
    go = torch.randn(B, S, O, generator=g).to(dev)
    y.backward(go)
    torch.cuda.synchronize()
    xn = x.detach().cpu().numpy().reshape(-1)
    anc = layer._detector_anchors.cpu().numpy()
    W = layer._weights.detach().cpu().numpy()
    pe = _full_pe(layer)
    geo = (B, S, n, n, pd, T, Nc, O)
    rout = oracle.fill_outputs_product(xn, xn, pe, anc, W, *geo, int_mode=True, int_rescaler=R)
    rxg, rpeg, rwg = oracle.propagate_product(xn, xn, pe, anc, W, go.cpu().numpy().reshape(-1), *geo,
                                              lr=1.0, int_mode=True, int_rescaler=R,
                                              w_grad=np.zeros(W.size, np.float32))
    for buf in (rout, rxg, rpeg, rwg):
        oracle.convert_int_to_float(buf, R)
    assert np.array_equal(y.detach().cpu().numpy().reshape(-1), rout)
    assert np.array_equal(x.grad.cpu().numpy().reshape(-1), rxg)
    assert np.array_equal(layer._weights.grad.cpu().numpy(), rwg)
    assert np.array_equal(layer._positional_embeddings.grad.cpu().numpy(), rpeg)


def test_layer_product_sparse_and_internal_policies(cuda_device):
    """Sparse: the same values as Dense, as a coalesced COO tensor.
    Internal: the weights move by the Dense gradient times -external_lr
    (within one fp32 rounding of each sum), and there is no weight grad."""
    from spiky_amd.lut.LUTLayer import GradientPolicy, GradientType
    dev = cuda_device
    B, S, n, T, Nc, O, pd = 2, 9, 10, 6, 4, 20, 3
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, S, n, generator=g).to(dev)
    go = torch.randn(B, S, O, generator=g).to(dev)
    grads = {}
    for kind in (GradientType.Dense, GradientType.Sparse):
        layer = _layer(dev, n, S, T, Nc, O, pd, policy=GradientPolicy(kind))
        layer(x).backward(go)
        grads[kind] = layer._weights.grad
    dense = grads[GradientType.Dense]
    sp = grads[GradientType.Sparse]
    assert sp.is_sparse
    assert torch.equal(sp.to_dense(), dense)
    layer = _layer(dev, n, S, T, Nc, O, pd, policy=GradientPolicy(GradientType.Internal))
    layer.set_external_learning_rate_hook(lambda w: 0.25)
    W0 = layer._weights.detach().clone()
    layer(x).backward(go)
    torch.cuda.synchronize()
    assert layer._weights.grad is None
    want = W0 - 0.25 * dense
    scale = float(W0.abs().max()) + 0.25 * float(dense.abs().max())
    assert torch.allclose(layer._weights.detach(), want, rtol=0, atol=4 * U * scale)


def test_transformer_product_attention(oracle, cuda_device):
    """LUTTransformer with concatenation_product=False: the attention layers
    run the product kernels.  The logits match the oracle chain whose
    attention outputs are the fp64 term sums rounded to fp32 (the GPU's own
    rounding), and every table receives a gradient."""
    from spiky_amd import LUTTransformer
    dev = cuda_device
    B, S, V, E = 2, 8, 16, 16
    model = LUTTransformer(vocab_size=V, embedding_dim=E, context_size=S, positional_dim=2, num_layers=2,
                           num_heads=2, n_detectors=3, n_anchors_per_detector=4,
                           n_anchors_per_detector_attention=3, concatenation_product=False, device=dev,
                           seed=11)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for p in (l._weights for l in model._lut_layers()):
            p.copy_((torch.randn(p.numel(), generator=g) * 0.05).to(dev))
    tokens = torch.randint(0, V, (B, S), generator=g).to(dev)
    logits = model(tokens)
    z = model.token_embedder.weight.detach().cpu().numpy()[tokens.cpu().numpy()].astype(np.float32)
    for block in model.layers:
        att = block["attention_lut"]
        T, Nc, pd = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
        zf = z.reshape(-1)
        s, _ = oracle.fill_outputs_product64(zf, zf, _full_pe(att), att._detector_anchors.cpu().numpy(),
                                             att._weights.detach().cpu().numpy(), B, S, E, E, pd, T, Nc,
                                             att._n_outputs)
        z = z + s.astype(np.float32).reshape(B, S, E)
        ffn = block["ffn"]
        Tf, Ncf = ffn._n_detectors, ffn._n_anchors_per_detector
        fi, _, _ = oracle.check_detectors(z.reshape(-1), ffn._detector_anchors.cpu().numpy(), B * S, E,
                                          Tf, Ncf)
        z = z + oracle.fill_outputs_fc(ffn._weights.detach().cpu().numpy(), fi, B * S, E, Tf,
                                       1 << Ncf).reshape(B, S, E)
    un = model.unembedder
    ui, _, _ = oracle.check_detectors(z.reshape(-1), un._detector_anchors.cpu().numpy(), B * S, E,
                                      un._n_detectors, un._n_anchors_per_detector)
    rlogits = oracle.fill_outputs_fc(un._weights.detach().cpu().numpy(), ui, B * S, V, un._n_detectors,
                                     1 << un._n_anchors_per_detector)
    np.testing.assert_allclose(logits.detach().cpu().numpy().reshape(-1), rlogits, rtol=1e-6, atol=1e-7)
    targets = torch.randint(0, V, (B, S), generator=g).to(dev)
    torch.nn.functional.cross_entropy(logits.reshape(-1, V), targets.reshape(-1)).backward()
    torch.cuda.synchronize()
    for l in model._lut_layers():
        assert l._weights.grad is not None and torch.isfinite(l._weights.grad).all()
    for block in model.layers:
        pg = block["attention_lut"]._positional_embeddings.grad
        assert pg is not None and torch.isfinite(pg).all()


# ---------------------------------------------------------------- sparse connectivity
def run_product_sparse(oracle, B, S, n, T, Nc, O, pd, sliced=False, int_rescaler=None, internal=False,
                       seed=0, lr=1.0, ext_lr=0.2):
    """Product mode over a random ragged CSR (empty neurons, repeated targets)
    against the oracle: int32 bit-exact; fp32 within the bounds above."""
    dev = torch.device("cuda:0")
    if sliced:
        pd = n
    int_mode = int_rescaler is not None
    print(f"[product sparse] B={B} S={S} n={n} T={T} Nc={Nc} O={O} pd={pd} sliced={sliced} "
          f"int={int_mode} internal={internal}", flush=True)
    x, pe, anc, _, g = product_inputs(seed, B, S, n, T, Nc, O, pd, sliced)
    rng = np.random.default_rng(seed + 100)
    E = 1 << Nc
    counts = rng.integers(0, 9, size=T * E)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    tg = rng.integers(0, O, size=int(off[-1])).astype(np.int32)
    W = (rng.standard_normal(tg.size) * 0.1).astype(np.float32)
    args = (2 * n + pd, O, T, Nc, 1, pd, 0, 4, 32)
    dm = LUTDataManagerF(*args) if int_rescaler is None else LUTDataManagerI(*args, int_rescaler)
    dm.register_synapse_meta(lr, -10.0, 10.0, 0.0, 0.0)
    dm.initialize_neurons(False)
    dm.set_lookup_connectivity(off, tg)
    dm.compile(True, torch.zeros(tg.size))
    dm.to_device(0)
    xd, ad, Wd, gd = (torch.from_numpy(v).to(dev) for v in (x, anc, W, g))
    ped = torch.from_numpy(pe).to(dev) if pd else None
    out = torch.zeros(B * S * O, device=dev)
    dm.forward_step_product(Wd, B, S, xd, xd, ad, out, n, n, sliced, 0.0, ped)
    xg = torch.zeros(B * S * n, device=dev)
    peg = torch.zeros((S - 1) * T * pd, device=dev) if pd else None
    W_before = W.copy()
    wg = None
    if internal:
        dm.backward_backprop_product(Wd, B, S, xd, xd, ad, gd, xg, xg, ext_lr, n, n, sliced, 0.0, None, ped, peg)
    else:
        wg = torch.zeros_like(Wd)
        dm.backward_backprop_product(Wd, B, S, xd, xd, ad, gd, xg, xg, -1.0, n, n, sliced, 0.0, wg, ped, peg)
    torch.cuda.synchronize()
    geo = (B, S, n, n, pd, T, Nc, O)
    eff_lr = lr * (-ext_lr if internal else 1.0)
    if int_mode:
        rout = oracle.fill_outputs_product_sparse(x, x, pe, anc, W, off, tg, *geo, sliced=sliced, int_mode=True,
                                                  int_rescaler=int_rescaler)
        rx, rp, rw = oracle.propagate_product_sparse(x, x, pe, anc, W, off, tg, g, *geo, sliced=sliced, lr=eff_lr,
                                                     int_mode=True, int_rescaler=int_rescaler)
        for buf in (rout, rx, rp, rw):
            if buf is not None:
                oracle.convert_int_to_float(buf, int_rescaler)
        assert np.array_equal(out.cpu().numpy(), rout)
        assert np.array_equal(xg.cpu().numpy(), rx)
        if pd:
            assert np.array_equal(peg.cpu().numpy(), rp)
        assert np.array_equal(wg.cpu().numpy(), rw)
        return
    s, a = oracle.fill_outputs_product_sparse(x, x, pe, anc, W, off, tg, *geo, sliced=sliced, bounds=True)
    n_fwd = T * S * int(counts.max())
    within(out.cpu().numpy(), s, a, n_fwd, "forward")
    r = oracle.propagate_product_sparse(x, x, pe, anc, W, off, tg, g, *geo, sliced=sliced, lr=eff_lr, bounds=True)
    within(xg.cpu().numpy(), *r["x"], 2 * T * S, "x_grad")
    if pd:
        within(peg.cpu().numpy(), *r["pe"], 2 * B * S, "pe_grad")
    n_w = B * S * (S - 1) // 2
    if internal:
        within(Wd.cpu().numpy(), W_before.astype(np.float64) + r["w"][0], r["w"][1] + np.abs(W_before), n_w,
               "weights (Internal)")
    else:
        within(wg.cpu().numpy(), *r["w"], n_w, "w_grad")
    assert np.abs(xg.cpu().numpy()).max() > 0


@pytest.mark.parametrize("sliced,pd", [(False, 0), (False, 3), (True, 0)])
def test_product_sparse_fp32(oracle, cuda_device, sliced, pd):
    run_product_sparse(oracle, B=2, S=10, n=8, T=4, Nc=4, O=12, pd=pd, sliced=sliced, seed=13)


@pytest.mark.parametrize("sliced", [False, True])
def test_product_sparse_int32_bit_exact(oracle, cuda_device, sliced):
    run_product_sparse(oracle, B=2, S=9, n=8, T=3, Nc=4, O=10, pd=2, sliced=sliced, int_rescaler=0.001, seed=14)


def test_product_sparse_internal_policy(oracle, cuda_device):
    run_product_sparse(oracle, B=2, S=8, n=6, T=3, Nc=3, O=9, pd=2, internal=True, lr=0.5, seed=15)


def test_product_sparse_conv2d_layer_autograd(oracle, cuda_device):
    """A sliced product-mode Conv2DLUTLayer with a lookup receptive field (sparse
    connectivity) through autograd."""
    from spiky_amd.lut.LUTLayer import Conv2DLUTLayer, SynapseMeta
    dev = cuda_device
    S = 5
    layer = Conv2DLUTLayer(input_shape=(4, 4), n_anchors_per_detector=3, detectors_shape=(2, 2),
                           output_kernel_shape=(2, 2), sequence_length=S, receptive_field_shape=(2, 2),
                           receptive_field_stride_shape=(1, 1), lut_receptive_field_shape=(4, 4),
                           lut_receptive_field_stride_shape=(2, 2), concatenation_product=False,
                           sliced_product_mode=True, positional_dim=16,
                           synapse_meta=SynapseMeta(initial_noise_level=1.0), _forward_group_size=3,
                           random_seed=3, device=dev)
    off, tg = layer._lut_dm.lookup_connectivity()
    T, Nc, O, n = layer.n_detectors(), layer.n_anchors_per_detector(), layer.n_outputs(), 16
    g = torch.Generator().manual_seed(6)
    B = 2
    x = torch.randn(B, S, 4, 4, generator=g).to(dev).requires_grad_(True)
    y = layer(x)
    go = torch.randn(B, S, 4, 4, generator=g).to(dev)
    y.backward(go)
    torch.cuda.synchronize()
    xn = x.detach().cpu().numpy().reshape(-1)
    anc = layer._detector_anchors.cpu().numpy()
    W = layer._weights.detach().cpu().numpy()
    pe = _full_pe(layer)
    geo = (B, S, n, n, 16, T, Nc, O)
    s, a = oracle.fill_outputs_product_sparse(xn, xn, pe, anc, W, off, tg, *geo, sliced=True, bounds=True)
    within(y.detach().cpu().numpy().reshape(-1), s, a, T * S * int(np.diff(off).max()), "forward")
    r = oracle.propagate_product_sparse(xn, xn, pe, anc, W, off, tg, go.cpu().numpy().reshape(-1), *geo,
                                        sliced=True, bounds=True)
    within(x.grad.cpu().numpy().reshape(-1), *r["x"], 2 * T * S, "x.grad")
    within(layer._weights.grad.cpu().numpy(), *r["w"], B * S * (S - 1) // 2, "weights.grad")
    within(layer._positional_embeddings.grad.cpu().numpy(), *r["pe"], 2 * B * S, "pe.grad")
    assert np.abs(r["w"][0]).max() > 0
