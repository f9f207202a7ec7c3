"""GPU parity at the layer level (LUTLayer / ProjectionLUTLayer through the
LUTForwardFN autograd function) and at BASELINE config 3's full size."""
import numpy as np
import pytest
import torch

from spiky_amd import GradientPolicy, GradientType, LUTLayer, ProjectionLUTLayer

pytestmark = pytest.mark.gpu


def _xg_close(gpu, cpu, B, I, rtol=1e-5):
    gpu = np.asarray(gpu).reshape(B, I)
    cpu = np.asarray(cpu).reshape(B, I)
    scale = np.abs(cpu).max(axis=1, keepdims=True) + 1e-30
    assert np.all(np.abs(gpu - cpu) <= rtol * scale)


def test_lut_layer_autograd(oracle, cuda_device):
    dev = cuda_device
    B, I, T, Nc, O = 32, 784, 256, 6, 10
    torch.manual_seed(0)
    layer = LUTLayer(I, Nc, T, O, random_seed=11).to(dev)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.01)
    x = torch.rand(B, 1, I, device=dev, requires_grad=True)
    y = layer(x)
    g = torch.randn_like(y)
    y.backward(g)
    E = 1 << Nc
    an = layer._detector_anchors.cpu().numpy()
    Wn = layer._weights.detach().cpu().numpy()
    xn = x.detach().cpu().numpy().reshape(-1)
    gn = g.cpu().numpy().reshape(-1)
    ridx, rmd, rmi = oracle.check_detectors(xn, an, B, I, T, Nc)
    rout = oracle.fill_outputs_fc(Wn, ridx, B, O, T, E)
    rxg = oracle.propagate_fc(Wn, gn, ridx, rmd, rmi, an, B, I, O, T, Nc, E)
    rwg = np.zeros(T * E * O, np.float32)
    oracle.gather_wgrad_fc(gn, ridx, rwg, B, O, T, E)
    assert np.array_equal(y.detach().cpu().numpy().reshape(-1), rout)
    _xg_close(x.grad.cpu().numpy(), rxg, B, I)
    assert np.array_equal(layer._weights.grad.cpu().numpy(), rwg)


def test_lut_layer_sparse_and_normalized_policies(oracle, cuda_device):
    dev = cuda_device
    B, I, T, Nc, O = 8, 64, 32, 4, 16
    for policy in (GradientPolicy(GradientType.Sparse), GradientPolicy(GradientType.Dense, normalized=True)):
        layer = LUTLayer(I, Nc, T, O, random_seed=3, weights_gradient_policy=policy).to(dev)
        with torch.no_grad():
            layer._weights.normal_(0.0, 0.01)
        x = torch.rand(B, 1, I, device=dev)
        y = layer(x)
        y.backward(torch.ones_like(y))
        E = 1 << Nc
        ridx, _, _ = oracle.check_detectors(x.cpu().numpy().reshape(-1),
                                            layer._detector_anchors.cpu().numpy(), B, I, T, Nc)
        rwg = np.zeros(T * E * O, np.float32)
        oracle.gather_wgrad_fc(np.ones(B * O, np.float32), ridx, rwg, B, O, T, E)
        got = layer._weights.grad
        if policy.type == GradientType.Sparse:
            # the converter's COO output: ascending indices (autograd's
            # accumulation into .grad does not keep the coalesced flag), and
            # the shared dense buffer left zeroed for the next step
            # (erase_input=True)
            assert got.is_sparse
            ind = got._indices()[0]
            assert bool((ind[1:] > ind[:-1]).all())
            assert torch.count_nonzero(layer._shared_context._weight_gradients_buffers[0]) == 0
        got = got.to_dense() if got.is_sparse else got
        if policy.normalized:
            rwg = rwg / max(np.abs(rwg).max(), 1e-16)
        np.testing.assert_allclose(got.cpu().numpy(), rwg, rtol=1e-6, atol=0)


def test_projection_layer_sparse_parity(oracle, cuda_device):
    dev = cuda_device
    torch.manual_seed(1)
    layer = ProjectionLUTLayer((28, 28), (24, 24), 5, 36, 8, (5, 5), (4, 4), random_seed=5).to(dev)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.01)
    B = 16
    T, Nc, I, O = layer.n_detectors(), 5, 784, 576
    E = 1 << Nc
    x = torch.rand(B, 1, 28, 28, device=dev)
    x = x * (torch.rand_like(x) > 0.8)
    x.requires_grad_(True)
    y = layer(x)
    g = torch.randn_like(y)
    y.backward(g)
    offs, tg = layer._lut_dm.lookup_connectivity()
    an = layer._detector_anchors.cpu().numpy()
    Wn = layer._weights.detach().cpu().numpy()
    xn = x.detach().cpu().numpy().reshape(-1)
    gn = g.cpu().numpy().reshape(-1)
    ridx, rmd, rmi = oracle.check_detectors(xn, an, B, I, T, Nc)
    rout = oracle.fill_outputs_sparse(Wn, ridx, offs, tg, B, O, T, E)
    maxg = layer._lut_dm.get_max_forward_groups_per_neuron()
    rxg = oracle.propagate_sparse(Wn, gn, ridx, rmd, rmi, an, offs, tg, B, I, O, T, Nc, E, 32, maxg)
    rwg = np.zeros(Wn.size, np.float32)
    oracle.gather_wgrad_sparse(gn, ridx, offs, tg, rwg, B, O, T, E)
    assert np.array_equal(y.detach().cpu().numpy().reshape(-1), rout)
    _xg_close(x.grad.cpu().numpy(), rxg, B, I)
    assert np.array_equal(layer._weights.grad.cpu().numpy(), rwg)


@pytest.mark.parametrize("geo", [
    # many tables on few inputs: the input-gradient adds summed in LDS first;
    # 6x6 projections give rows of 36 entries, two forward groups
    dict(inp=(12, 12), out=(24, 24), groups=64, tables=16, field=(5, 5), proj=(6, 6), B=40),
    # rows of 1..4 entries (one slot a lane), inputs outnumbering the adds
    dict(inp=(32, 32), out=(16, 16), groups=9, tables=8, field=(7, 7), proj=(2, 2), B=24),
    # forward groups of 64 entries, rows of 12..36 (median 24: 8 slots a lane),
    # so the longest rows take two passes
    dict(inp=(16, 16), out=(10, 10), groups=25, tables=12, field=(5, 5), proj=(6, 6), B=17, fgs=64),
])
def test_projection_layer_sparse_backward_shapes(oracle, cuda_device, geo):
    """The fp32 input gradient over uniform rows (four lanes per table and
    group, entry slots for a median row, LDS-summed adds where inputs are few)
    against the CPU restatement, with the weight gradient bit-exact."""
    dev = cuda_device
    torch.manual_seed(3)
    fgs = geo.get("fgs", 32)
    layer = ProjectionLUTLayer(geo["inp"], geo["out"], 5, geo["groups"], geo["tables"], geo["field"], geo["proj"],
                               random_seed=9, _forward_group_size=fgs).to(dev)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.01)
    B = geo["B"]
    T, Nc = layer.n_detectors(), 5
    I, O = geo["inp"][0] * geo["inp"][1], geo["out"][0] * geo["out"][1]
    E = 1 << Nc
    x = torch.rand(B, 1, *geo["inp"], device=dev)
    x = (x * (torch.rand_like(x) > 0.5)).requires_grad_(True)
    y = layer(x)
    g = torch.randn_like(y)
    y.backward(g)
    offs, tg = layer._lut_dm.lookup_connectivity()
    an = layer._detector_anchors.cpu().numpy()
    Wn = layer._weights.detach().cpu().numpy()
    xn = x.detach().cpu().numpy().reshape(-1)
    gn = g.cpu().numpy().reshape(-1)
    ridx, rmd, rmi = oracle.check_detectors(xn, an, B, I, T, Nc)
    maxg = layer._lut_dm.get_max_forward_groups_per_neuron()
    rxg = oracle.propagate_sparse(Wn, gn, ridx, rmd, rmi, an, offs, tg, B, I, O, T, Nc, E, fgs, maxg)
    rwg = np.zeros(Wn.size, np.float32)
    oracle.gather_wgrad_sparse(gn, ridx, offs, tg, rwg, B, O, T, E)
    assert np.array_equal(y.detach().cpu().numpy().reshape(-1), oracle.fill_outputs_sparse(Wn, ridx, offs, tg, B, O, T, E))
    _xg_close(x.grad.cpu().numpy(), rxg, B, I)
    assert np.array_equal(layer._weights.grad.cpu().numpy(), rwg)


@pytest.mark.parametrize("B", [48, 70, 130])
@pytest.mark.parametrize("int_sums", [False, True])
@pytest.mark.parametrize("Nc", [5, 9])
def test_projection_layer_sparse_forward_wide_batches(oracle, cuda_device, B, int_sums, Nc):
    """The sparse forward at batches of 48 and more (a wavefront per output and
    64 samples over table-major keys: one byte a key at 32 rows, two at 512),
    with partly filled wavefronts and outputs no synapse reaches, in fp32 and
    int32 sums: bit-exact against the CPU restatement."""
    dev = cuda_device
    kw = dict(summation_dtype=torch.int32, _int_rescaler=0.37) if int_sums else {}
    layer = ProjectionLUTLayer((20, 20), (16, 16), Nc, 20, 6, (5, 5), (4, 4), random_seed=11, **kw).to(dev)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.05)
    T, I, O = layer.n_detectors(), 400, 256
    E = 1 << Nc
    x = torch.rand(B, 1, 20, 20, device=dev)
    layer.eval()
    with torch.no_grad():
        y = layer(x)
    offs, tg = layer._lut_dm.lookup_connectivity()
    assert np.bincount(np.asarray(tg), minlength=O).min() == 0    # some outputs have empty lists
    ridx, _, _ = oracle.check_detectors(x.cpu().numpy().reshape(-1), layer._detector_anchors.cpu().numpy(),
                                        B, I, T, Nc)
    Wn = layer._weights.detach().cpu().numpy()
    rout = oracle.fill_outputs_sparse(Wn, ridx, offs, tg, B, O, T, E, int_mode=int_sums,
                                      int_rescaler=0.37 if int_sums else 1.0)
    if int_sums:
        oracle.convert_int_to_float(rout, 0.37)    # the restatement leaves the int32 payloads
    assert np.array_equal(y.cpu().numpy().reshape(-1), rout)


@pytest.mark.parametrize("int_sums", [False, True])
@pytest.mark.parametrize("overwrite", [False, True])
@pytest.mark.parametrize("B", [70, 100])
def test_projection_sparse_wgrad_modes(oracle, cuda_device, int_sums, overwrite, B):
    """The sparse weight gradient over uniform rows through the data manager --
    a thread per synapse (70 samples over 32 rows) or per synapse slot of four
    rows walking their samples in bucket order (100 samples) -- written over or
    added to a buffer holding other values, in fp32 and int32 sums (where the
    buffer holds int32 payloads and each row ends converted), bit-exact against
    the CPU restatement."""
    dev = cuda_device
    R = 0.37
    kw = dict(summation_dtype=torch.int32, _int_rescaler=R) if int_sums else {}
    layer = ProjectionLUTLayer((16, 16), (12, 12), 5, 16, 8, (5, 5), (4, 4), random_seed=4, **kw).to(dev)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.05)
    dm = layer._lut_dm
    T, I, O, E = layer.n_detectors(), 256, 144, 32
    torch.manual_seed(6)
    x = torch.rand(B * I, device=dev)
    out = torch.zeros(B * O, device=dev)
    li = torch.zeros(B * T, dtype=torch.int32, device=dev)
    md = torch.zeros(B * T, device=dev)
    mi = torch.zeros(B * T, dtype=torch.int32, device=dev)
    dm.forward_step(layer._weights, B, x, layer._detector_anchors, out, li, 0.0,
                    w_min_anchor_deltas=md, w_min_anchor_delta_indices=mi)
    g = torch.randn(B * O, device=dev)
    xg = torch.zeros(B * I, device=dev)
    W = layer._weights.numel()
    if int_sums:
        init = torch.randint(-5000, 5000, (W,), dtype=torch.int32).view(torch.float32)
    else:
        init = torch.randn(W)
    wg = init.clone().to(dev)
    dm.backward_backprop(layer._weights, B, g, layer._detector_anchors, li, md, mi, xg, -1.0, wg,
                         overwrite_weights_gradients=overwrite)
    offs, tg = dm.lookup_connectivity()
    rt = np.zeros(W, np.float32) if overwrite else init.numpy().copy()
    oracle.gather_wgrad_sparse(g.cpu().numpy(), li.cpu().numpy(), offs, tg, rt, B, O, T, E,
                               int_mode=int_sums, int_rescaler=R)
    if int_sums:
        oracle.convert_int_to_float(rt, R)
    assert np.array_equal(wg.cpu().numpy().view(np.int32), rt.view(np.int32))


def test_projection_layer_built_on_device(cuda_device):
    """A ProjectionLUTLayer constructed with device=cuda grows its connectivity
    on the host and gives the same layer as one built on the host and moved."""
    dev = cuda_device
    kw = dict(random_seed=7)
    a = ProjectionLUTLayer((16, 16), (12, 12), 4, 9, 4, (5, 5), (4, 4), device=dev, **kw)
    b = ProjectionLUTLayer((16, 16), (12, 12), 4, 9, 4, (5, 5), (4, 4), **kw).to(dev)
    assert torch.equal(a._detector_anchors.cpu(), b._detector_anchors.cpu())
    oa, ta = a._lut_dm.lookup_connectivity()
    ob, tb = b._lut_dm.lookup_connectivity()
    assert np.array_equal(np.asarray(oa), np.asarray(ob)) and np.array_equal(np.asarray(ta), np.asarray(tb))
    with torch.no_grad():
        b._weights.copy_(a._weights)
    x = torch.rand(3, 1, 16, 16, device=dev)
    assert torch.equal(a(x), b(x))


def fold_blocks(B, T, O, dgs=32):
    """Blocks of dgs tables the table-major fp32 forward sums in fp64 before one
    commit when ordered sums are off: enough to leave about 1024 work units of
    (block group, 32-column slice, 1024-sample chunk) -- the library's rule,
    restated so a change of it shows here."""
    n_blocks = -(-T // dgs)
    spt = 1 if B <= 128 else 2 if B <= 256 else 4 if B <= 512 else 8
    units = n_blocks * -(-B // (128 * spt)) * -(-O // 32)
    return max(1, min(n_blocks, units // 1024))


@pytest.mark.parametrize("ordered", [False, True])
def test_config3_full_size(oracle, cuda_device, ordered):
    """BASELINE config 3 at its real size.  The oracle cannot hold the whole
    problem in seconds, so parity is checked on slices the arithmetic allows:
    every sample's forward output depends only on its own rows (gathered
    host-side into an E=1 table), every table's weight gradient only on that
    table, every sample's input gradient only on its main and flipped rows.
    With ordered sums the output is the reference CPU path's, bit for bit;
    by default (eight blocks folded into one fp64 sum) it is the oracle's with
    256-table blocks bit for bit, and within 1e-5 of the ordered result."""
    dev = cuda_device
    B, I, T, Nc, O = 1024, 4096, 8192, 8, 1024
    E = 1 << Nc
    from spiky_amd import LUTDataManagerF
    dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, 32, 32)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    dm.set_ordered_sums(ordered)
    fold = 1 if ordered else fold_blocks(B, T, O)
    assert ordered or fold == 8
    gen = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(B * I, device=dev, generator=gen)
    W = torch.randn(T * E * O, device=dev, generator=gen) * 0.01
    go = torch.randn(B * O, device=dev, generator=gen)
    ga = torch.Generator().manual_seed(4)
    anchors = torch.stack([torch.randperm(I, generator=ga)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    ad = anchors.to(dev)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    md = torch.empty(B * T, device=dev)
    mi = torch.empty(B * T, dtype=torch.int32, device=dev)
    print("[config3] forward", flush=True)
    dm.forward_step(W, B, x, ad, out, idx, 0.0, None, md, mi)
    xg = torch.zeros(B * I, device=dev)
    wg = torch.empty(T * E * O, device=dev)
    print("[config3] backward", flush=True)
    dm.backward_backprop(W, B, go, ad, idx, md, mi, xg, -1.0, wg, None, overwrite_weights_gradients=True)
    torch.cuda.synchronize()
    # every table's gradient rows sum to the batch's gradient sum (each sample hits one row per table)
    colsum = go.view(B, O).double().sum(0)
    per_table = wg.view(T, E, O).double().sum(1)
    assert torch.allclose(per_table, colsum.expand(T, O), rtol=0, atol=1e-3)
    xs = x.view(B, I)
    samples = [0, 513, B - 1]
    an = anchors.numpy()
    ridx, rmd, rmi = oracle.check_detectors(xs[samples].cpu().numpy().reshape(-1), an, len(samples), I, T, Nc)
    assert np.array_equal(idx.view(B, T)[samples].cpu().numpy().reshape(-1), ridx)
    assert np.array_equal(md.view(B, T)[samples].cpu().numpy().reshape(-1), rmd)
    assert np.array_equal(mi.view(B, T)[samples].cpu().numpy().reshape(-1), rmi)
    Wv = W.view(T, E, O)
    tt = torch.arange(T, device=dev)
    for s in samples:
        rows = Wv[tt, idx.view(B, T)[s].long()].cpu().numpy().reshape(-1)       # [T][O], E=1
        r = oracle.fill_outputs_fc(rows, np.zeros((1, T), np.int32), 1, O, T, 1, dgs=32 * fold)
        got = out.view(B, O)[s].cpu().numpy()
        assert np.array_equal(got, r)
        r32 = oracle.fill_outputs_fc(rows, np.zeros((1, T), np.int32), 1, O, T, 1, dgs=32)
        assert np.abs(got - r32).max() <= 1e-5 * np.abs(r32).max()
        li = idx.view(B, T)[s].long()
        alt = li ^ (1 << mi.view(B, T)[s].long())
        pair = torch.stack([Wv[tt, li], Wv[tt, alt]], 1).cpu().numpy().reshape(-1)  # [T][2][O]
        a_sub = anchors.view(T, Nc, 2)[torch.arange(T), mi.view(B, T)[s].cpu().long()].numpy().reshape(-1)
        rxg = oracle.propagate_fc(pair, go.view(B, O)[s].cpu().numpy(), np.zeros(T, np.int32),
                                  md.view(B, T)[s].cpu().numpy(), np.zeros(T, np.int32), a_sub, 1, I,
                                  O, T, 1, 2, ogs=32)
        _xg_close(xg.view(B, I)[s].cpu().numpy(), rxg, 1, I)
    for t in (0, 4097, T - 1):
        r = np.zeros(E * O, np.float32)
        oracle.gather_wgrad_fc(go.cpu().numpy(), idx.view(B, T)[:, t].cpu().numpy().copy(), r, B, O, 1, E)
        assert np.array_equal(wg.view(T, E * O)[t].cpu().numpy(), r)


def test_pickle_checkpoint_roundtrip(cuda_device):
    """A trained layer refuses to pickle on the device (lut.cu:1410-1412); moved
    to the CPU it pickles, and restored on the device it gives the same
    outputs and gradients bit for bit."""
    import pickle
    dev = cuda_device
    B, I, T, Nc, O = 32, 96, 64, 5, 24
    layer = LUTLayer(I, Nc, T, O, random_seed=9).to(dev)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.01)
    with pytest.raises(RuntimeError, match="net must be on CPU before serialization"):
        pickle.dumps(layer)
    x = torch.randn(B, 1, I, device=dev, requires_grad=True)
    g = torch.randn(B, 1, O, device=dev)
    y1 = layer(x)
    y1.backward(g)
    wg1, xg1 = layer._weights.grad.clone(), x.grad.clone()
    blob = pickle.dumps(layer.to("cpu"))
    restored = pickle.loads(blob).to(dev)
    x.grad = None
    y2 = restored(x)
    y2.backward(g)
    assert torch.equal(y1, y2)
    assert torch.equal(wg1, restored._weights.grad)
    assert torch.equal(xg1, x.grad)
