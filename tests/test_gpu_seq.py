"""GPU parity of the sequence-concat LUT path (LUTTransformer attention)
against the CPU oracle (oracle/lut_oracle.c, restating
lut_runtime_kernels_logic.proto:1589-1904,3629-4045).

Bars:
  * lookup indices, min margins and indices (tokens and positions): bit-exact;
  * forward output: bit-exact (pairs summed in fp64, one fp32 commit per
    table in ascending order, as the reference CPU path);
  * int32 summation: every accumulator bit-exact;
  * fp32 weight gradient: the reference GPU adds it with atomics in any order,
    so it is bit-exact only when g is integer-valued (order-free sums), and
    otherwise within the fp32 summation bound n * 2^-24 * sum|terms|;
  * fp32 input and positional gradients: |gpu - cpu| <= 1e-5 * max|row| plus
    the sub-EPS terms the reference drops per (pair, table, block), where cpu
    is the oracle's terms summed in fp64 (its fp32 partial sums are the
    reference's own rounding noise, pinned in test_oracle_seq_pins.py).
"""
import numpy as np
import pytest
import torch

from spiky_amd import LUTDataManagerF, LUTDataManagerI

pytestmark = pytest.mark.gpu


def make_seq_dm(I, O, T, Nc, S, Npe, fgs=32, bgs=32, int_rescaler=None, lr=1.0):
    if int_rescaler is None:
        dm = LUTDataManagerF(I, O, T, Nc, S, Npe, 0, fgs, bgs)
    else:
        dm = LUTDataManagerI(I, O, T, Nc, S, Npe, 0, fgs, bgs, int_rescaler)
    dm.register_synapse_meta(lr, -10.0, 10.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    return dm


def seq_inputs(seed, B, S, I, T, Nc, Npe, O, int_grad=False):
    g = torch.Generator().manual_seed(seed)
    E = 1 << (2 * Nc + Npe)
    x = torch.randn(B * S * I, generator=g)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    W = torch.randn(T * E * O, generator=g) * 0.01
    pe = torch.rand((S - 1) * T * max(Npe, 1), generator=g) * 2 - 1
    if int_grad:
        go = torch.randint(-3, 4, (B * S * O,), generator=g).to(torch.float32)
    else:
        go = torch.randn(B * S * O, generator=g)
    return x, anchors, W, pe[: (S - 1) * T * Npe], go


def close_rows(gpu, cpu, rows, n_terms):
    gpu = np.asarray(gpu).reshape(rows, -1)
    cpu = np.asarray(cpu).reshape(rows, -1)
    bound = 1e-5 * np.abs(cpu).max(axis=1, keepdims=True) + n_terms * 1e-17
    err = np.abs(gpu - cpu)
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"


def run_seq(oracle, B, S, I, T, Nc, Npe, O, fgs=32, bgs=32, seed=0, int_rescaler=None, lr=1.0,
            int_grad=False, internal=False, inputs=None, accumulate=False):
    dev = torch.device("cuda:0")
    int_mode = int_rescaler is not None
    x, anchors, W, pe, go = inputs if inputs is not None else seq_inputs(seed, B, S, I, T, Nc, Npe, O, int_grad)
    dm = make_seq_dm(I, O, T, Nc, S, Npe, fgs, bgs, int_rescaler, lr)
    print(f"[seq] B={B} S={S} I={I} T={T} Nc={Nc} Npe={Npe} O={O} int={int_mode} internal={internal}",
          flush=True)
    Wd, xd, ad, ged = W.to(dev), x.to(dev), anchors.to(dev), go.to(dev)
    ped = pe.to(dev) if Npe else None
    n = B * S * T
    out = torch.zeros(B * S * O, device=dev)
    idx = torch.empty(n, dtype=torch.int32, device=dev)
    md = torch.empty(n, device=dev)
    mi = torch.empty(n, dtype=torch.int32, device=dev)
    npe = (S - 1) * T
    pli = torch.empty(npe, dtype=torch.int32, device=dev) if Npe else None
    pmd = torch.empty(npe, device=dev) if Npe else None
    pmi = torch.empty(npe, dtype=torch.int32, device=dev) if Npe else None
    dm.forward_step_concat(Wd, B, xd, ad, out, idx, 0.0, ped, pli, md, mi, pmd, pmi)
    xg = torch.zeros(B * S * I, device=dev)
    peg = torch.zeros(npe * Npe, device=dev) if Npe else None
    if internal:
        W_before = Wd.clone()
        dm.backward_backprop_concat(Wd, B, ged, ad, idx, md, mi, xg, 0.1, pli, pmd, pmi, peg, None)
        wg = None
    elif accumulate:
        # the caller's gradient buffer already holds values (every 7th one -0.0):
        # the kernels add to it, and rows no pair reaches keep their bits
        gp = torch.Generator().manual_seed(seed + 100)
        prefill = torch.randn(Wd.numel(), generator=gp) * 0.01
        prefill[::7] = -0.0
        wg = prefill.to(dev)
        dm.backward_backprop_concat(Wd, B, ged, ad, idx, md, mi, xg, -1.0, pli, pmd, pmi, peg, wg,
                                    overwrite_weights_gradients=False)
    else:
        wg = torch.empty_like(Wd)
        dm.backward_backprop_concat(Wd, B, ged, ad, idx, md, mi, xg, -1.0, pli, pmd, pmi, peg, wg,
                                    overwrite_weights_gradients=True)
    torch.cuda.synchronize()

    xn, an, Wn, gn = x.numpy(), anchors.numpy(), W.numpy(), go.numpy()
    ridx, rmd, rmi = oracle.check_detectors(xn, an, B * S, I, T, Nc)
    rpli = rpmd = rpmi = None
    if Npe:
        rpli, rpmd, rpmi = oracle.check_pe(pe.numpy(), S, T, Npe)
    rout = oracle.fill_outputs_seq(Wn, ridx, rpli, B, O, T, S, Nc, Npe, int_mode=int_mode,
                                   int_rescaler=int_rescaler or 1.0)
    # fp32 summation: the oracle's terms summed in fp64 (the reference CPU path
    # rounds every partial sum to fp32, an error that grows with S * T terms)
    rxg, rpeg = oracle.propagate_seq(Wn, gn, ridx, rmd, rmi, rpli, rpmd, rpmi, an, B, I, O, T, S, Nc,
                                     Npe, ogs=fgs, int_mode=int_mode, int_rescaler=int_rescaler or 1.0,
                                     acc64=not int_mode)
    if int_mode:
        oracle.convert_int_to_float(rout, int_rescaler)
        oracle.convert_int_to_float(rxg, int_rescaler)
        if Npe:
            oracle.convert_int_to_float(rpeg, int_rescaler)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(md.cpu().numpy(), rmd)
    assert np.array_equal(mi.cpu().numpy(), rmi)
    if Npe:
        assert np.array_equal(pli.cpu().numpy(), rpli)
        assert np.array_equal(pmd.cpu().numpy(), rpmd)
        assert np.array_equal(pmi.cpu().numpy(), rpmi)
    assert np.array_equal(out.cpu().numpy(), rout)
    n_ob = (O + fgs - 1) // fgs
    if int_mode:
        assert np.array_equal(xg.cpu().numpy(), rxg)
        if Npe:
            assert np.array_equal(peg.cpu().numpy(), rpeg)
    else:
        close_rows(xg.cpu().numpy(), rxg, B * S, S * T * n_ob)
        if Npe:
            pg, rp = peg.cpu().numpy(), rpeg
            assert np.abs(pg - rp).max() <= 1e-5 * max(np.abs(rp).max(), 1e-30)
    # weight gradient (or the in-place update)
    ext = 0.1 if internal else -1.0
    if internal:
        rW = Wn.copy()
        oracle.gather_wgrad_seq(gn, ridx, rpli, rW, B, O, T, S, Nc, Npe, ogs=fgs, first_meta_lr=lr,
                                external_lr=np.float32(ext))
        got, ref, base = Wd.cpu().numpy(), rW, W_before.cpu().numpy()
    elif accumulate:
        base = prefill.numpy()
        rwg = base.copy()
        oracle.gather_wgrad_seq(gn, ridx, rpli, rwg, B, O, T, S, Nc, Npe, ogs=fgs, first_meta_lr=lr)
        got, ref = wg.cpu().numpy(), rwg
        reach = np.zeros(Wn.size, np.float32)
        oracle.gather_wgrad_seq(np.ones_like(gn), ridx, rpli, reach, B, O, T, S, Nc, Npe, ogs=fgs,
                                first_meta_lr=1.0)
        untouched = reach == 0
        assert untouched.any() and (~untouched).any()
        assert np.array_equal(got[untouched].view(np.uint32), base[untouched].view(np.uint32))
    else:
        rwg = np.zeros(Wn.size, np.float32)
        oracle.gather_wgrad_seq(gn, ridx, rpli, rwg, B, O, T, S, Nc, Npe, ogs=fgs, first_meta_lr=lr,
                                int_mode=int_mode, int_rescaler=int_rescaler or 1.0)
        if int_mode:
            oracle.convert_int_to_float(rwg, int_rescaler)
        got, ref, base = wg.cpu().numpy(), rwg, 0.0
    if int_mode or int_grad:
        assert np.array_equal(got, ref)
    else:
        # fp32 sums of the same terms in another order: n * 2^-24 * sum|terms|
        mag = np.zeros(Wn.size, np.float32)
        oracle.gather_wgrad_seq(np.abs(gn), ridx, rpli, mag, B, O, T, S, Nc, Npe, ogs=fgs,
                                first_meta_lr=abs(lr * (0.1 if internal else 1.0)))
        bound = (B * S) * 2.0 ** -24 * (mag + np.abs(base)) + 1e-30
        assert np.all(np.abs(got - ref) <= bound), f"max excess {np.max(np.abs(got - ref) - bound)}"


def test_seq_small_with_pe(oracle, cuda_device):
    run_seq(oracle, 3, 9, 20, 5, 3, 2, 40, seed=1)


def test_seq_integer_gradients_exact(oracle, cuda_device):
    run_seq(oracle, 3, 9, 20, 5, 3, 2, 40, seed=2, int_grad=True)


def test_seq_no_positional(oracle, cuda_device):
    run_seq(oracle, 2, 12, 16, 4, 3, 0, 64, seed=3)


def test_seq_two_tiles_wide_rows(oracle, cuda_device):
    # S > 32 (several pair tiles in the reference order), 256 outputs (4 per lane)
    run_seq(oracle, 2, 40, 24, 3, 3, 3, 256, seed=4)


def test_seq_attention_layer_shape(oracle, cuda_device):
    # the config-5 attention layer's per-table shape (S = 256, Nc = 6, Npe = 4,
    # 2^10-row sub-tables, O = 256) at a batch and table count the oracle
    # finishes in seconds: LDS-sliced forward, the grouped backward (one
    # workgroup per (table, Q, group of 8 K values), k_propagate_seq_grp)
    run_seq(oracle, 2, 256, 64, 4, 6, 4, 256, seed=11)


def test_seq_one_bucket_chunks(oracle, cuda_device):
    # all-zero inputs put every (b, s) of a table in one Q bucket: more items
    # than one sorted chunk of the forward (1024), many weight-gradient
    # batches, and rows past one staged key chunk (8192)
    B, S, I, T, Nc, Npe, O = 160, 64, 16, 2, 3, 2, 64
    x, anchors, W, pe, go = seq_inputs(12, B, S, I, T, Nc, Npe, O)
    x.zero_()
    run_seq(oracle, B, S, I, T, Nc, Npe, O, seed=12, inputs=(x, anchors, W, pe, go))


def test_seq_one_bucket_chunks_partial_slice(oracle, cuda_device):
    # one Q bucket of 10240 items (ten sorted chunks of the forward) with 96
    # outputs: the first 64-column slice is staged by LDS DMA, the second runs
    # past the row's end and is staged through registers with zeros past it
    B, S, I, T, Nc, Npe, O = 160, 64, 16, 2, 3, 2, 96
    x, anchors, W, pe, go = seq_inputs(19, B, S, I, T, Nc, Npe, O)
    x.zero_()
    run_seq(oracle, B, S, I, T, Nc, Npe, O, seed=19, inputs=(x, anchors, W, pe, go))


def test_seq_many_rows_few_tables(oracle, cuda_device):
    # B*S >= 2048 rows over a few tables: the bucket sorts run a workgroup per
    # table (per-wave runs of the rows, scanned in (bucket, wave) order)
    run_seq(oracle, 16, 160, 32, 3, 4, 3, 64, seed=18)


@pytest.mark.parametrize("shape", [(3, 100, 48, 3, 5, 5, 128), (2, 513, 32, 2, 5, 6, 64),
                                   (2, 30, 16, 3, 1, 0, 64)])
def test_seq_grouped_input_gradient(oracle, cuda_device, shape):
    # the LDS-grouped input-gradient pass at shapes besides the attention
    # layer's: four K groups of 128-output rows (K flips of the high bits cross
    # groups), the longest sequence it takes (512 distances, 6 positional
    # bits, four groups of 64-output rows), and a sub-table below one KiB
    B, S, I, T, Nc, Npe, O = shape
    run_seq(oracle, B, S, I, T, Nc, Npe, O, seed=30 + Nc)


def test_seq_many_buckets_table_order(oracle, cuda_device):
    # more (table, Q) buckets than the largest-first order sorts in its one
    # workgroup (4100 x 16 > 65536): the forward and the weight gradient then
    # take them in table order, 64-column slices (the weight gradient's wide pass)
    run_seq(oracle, 2, 8, 16, 4100, 4, 0, 64, seed=40)


def test_seq_attention_layer_shape_int32(oracle, cuda_device):
    run_seq(oracle, 2, 256, 64, 4, 6, 4, 256, seed=13, int_rescaler=0.25)


def test_seq_one_bucket_chunks_int32(oracle, cuda_device):
    B, S, I, T, Nc, Npe, O = 160, 64, 16, 2, 3, 2, 64
    x, anchors, W, pe, go = seq_inputs(14, B, S, I, T, Nc, Npe, O)
    x.zero_()
    run_seq(oracle, B, S, I, T, Nc, Npe, O, seed=14, int_rescaler=0.5, inputs=(x, anchors, W, pe, go))


@pytest.mark.parametrize("shape", [(2, 20, 16, 3, 3, 2, 16), (2, 24, 16, 2, 6, 6, 32)])
def test_seq_narrow_forward_slices(oracle, cuda_device, shape):
    # 16-column forward slices (O = 16) and 8-column slices (2^12-row
    # sub-tables): one column a lane in the LDS-staged forward
    B, S, I, T, Nc, Npe, O = shape
    run_seq(oracle, B, S, I, T, Nc, Npe, O, seed=17 + Nc)


def test_seq_odd_outputs_and_groups(oracle, cuda_device):
    # O not a multiple of 4: exact decomposition path; odd group sizes
    run_seq(oracle, 2, 10, 12, 3, 2, 2, 37, fgs=8, bgs=5, seed=5)


def test_seq_int32_summation(oracle, cuda_device):
    run_seq(oracle, 2, 10, 16, 4, 3, 2, 48, seed=6, int_rescaler=0.5)


def test_seq_internal_policy(oracle, cuda_device):
    run_seq(oracle, 2, 9, 16, 3, 3, 2, 32, seed=7, lr=0.5, internal=True)


def test_seq_internal_policy_wide_rows(oracle, cuda_device):
    # 64-column weight-gradient slices (16-byte row pieces) adding into the weights
    run_seq(oracle, 2, 40, 16, 3, 3, 2, 64, seed=15, lr=0.5, internal=True)


def test_seq_accumulate_into_gradient(oracle, cuda_device):
    # the attention layer's per-table shape, adding into a filled gradient buffer
    run_seq(oracle, 2, 256, 64, 2, 6, 4, 256, seed=16, accumulate=True)


def test_seq_eval_mode(oracle, cuda_device):
    dev = cuda_device
    B, S, I, T, Nc, Npe, O = 2, 7, 12, 3, 2, 2, 24
    x, anchors, W, pe, _ = seq_inputs(8, B, S, I, T, Nc, Npe, O)
    dm = make_seq_dm(I, O, T, Nc, S, Npe)
    out = torch.zeros(B * S * O, device=dev)
    idx = torch.empty(B * S * T, dtype=torch.int32, device=dev)
    pli = torch.empty((S - 1) * T, dtype=torch.int32, device=dev)
    dm.forward_step_concat(W.to(dev), B, x.to(dev), anchors.to(dev), out, idx, 0.0, pe.to(dev), pli)
    ridx = oracle.check_detectors(x.numpy(), anchors.numpy(), B * S, I, T, Nc, train=False)
    rpli = oracle.check_pe(pe.numpy(), S, T, Npe, train=False)
    rout = oracle.fill_outputs_seq(W.numpy(), ridx, rpli, B, O, T, S, Nc, Npe)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(pli.cpu().numpy(), rpli)
    assert np.array_equal(out.cpu().numpy(), rout)


def test_seq_layer_autograd(oracle, cuda_device):
    """LUTLayer with sequence_length > 1 through torch autograd (reference
    LUTForwardFN, LUTLayer.py:1117-1181): output, input gradient, weight
    gradient and positional-embedding gradient against the oracle."""
    from spiky_amd import LUTLayer
    dev = cuda_device
    B, S, I, T, Nc, Npe, O = 2, 11, 16, 4, 3, 2, 32
    g = torch.Generator().manual_seed(9)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    layer = LUTLayer(I, Nc, T, O, sequence_length=S, positional_dim=Npe, _explicit_anchors=anchors,
                     device=dev, random_seed=3)
    with torch.no_grad():
        layer._weights.copy_((torch.randn(layer._weights.numel(), generator=g) * 0.01).to(dev))
    x = torch.randn(B, S, I, generator=g).to(dev).requires_grad_(True)
    y = layer(x)
    go = torch.randint(-3, 4, (B, S, O), generator=g).to(torch.float32).to(dev)
    y.backward(go)
    torch.cuda.synchronize()
    Wn = layer._weights.detach().cpu().numpy()
    pe = layer._positional_embeddings.detach().cpu().numpy()
    ridx, rmd, rmi = oracle.check_detectors(x.detach().cpu().numpy().reshape(-1), anchors.numpy(), B * S, I, T, Nc)
    rpli, rpmd, rpmi = oracle.check_pe(pe, S, T, Npe)
    rout = oracle.fill_outputs_seq(Wn, ridx, rpli, B, O, T, S, Nc, Npe)
    assert np.array_equal(y.detach().cpu().numpy().reshape(-1), rout)
    gn = go.cpu().numpy().reshape(-1)
    rxg, rpeg = oracle.propagate_seq(Wn, gn, ridx, rmd, rmi, rpli, rpmd, rpmi, anchors.numpy(), B, I, O,
                                     T, S, Nc, Npe)
    close_rows(x.grad.cpu().numpy(), rxg, B * S, S * T)
    pg = layer._positional_embeddings.grad.cpu().numpy()
    assert np.abs(pg - rpeg).max() <= 1e-5 * max(np.abs(rpeg).max(), 1e-30)
    rwg = np.zeros(Wn.size, np.float32)
    oracle.gather_wgrad_seq(gn, ridx, rpli, rwg, B, O, T, S, Nc, Npe)
    assert np.array_equal(layer._weights.grad.cpu().numpy(), rwg)


def test_seq_degenerate_anchors_int32(oracle, cuda_device):
    """Explicit anchors drawn with repetition, a quarter comparing an input with
    itself (Δ = 0 on both sides of the concatenation: bit 0, and the two pushes
    of the min-margin pair cancel), in int32 summation, where every output and
    gradient is bit-exact whatever the order of the pushes."""
    B, S, I, T, Nc, Npe, O = 2, 20, 12, 4, 3, 2, 32
    x, anchors, W, pe, go = seq_inputs(51, B, S, I, T, Nc, Npe, O)
    g = torch.Generator().manual_seed(52)
    a = torch.randint(0, I, (T * Nc, 2), generator=g, dtype=torch.int32)
    a[::4, 1] = a[::4, 0]
    run_seq(oracle, B, S, I, T, Nc, Npe, O, int_rescaler=0.5,
            inputs=(x, a.flatten().contiguous(), W, pe, go))


@pytest.mark.parametrize("int_rescaler", [None, 0.5])
def test_seq_shortest_sequences(oracle, cuda_device, int_rescaler):
    """S = 2 and 3: one and three causal pairs a sequence, a single distance."""
    run_seq(oracle, 4, 2, 8, 3, 2, 1, 16, seed=70, int_rescaler=int_rescaler)
    run_seq(oracle, 3, 3, 8, 3, 2, 1, 64, seed=71, int_rescaler=int_rescaler)


def test_seq_past_the_grouped_propagate(oracle, cuda_device):
    """S = 520, past the 513 positions the grouped input-gradient pass takes:
    the pair-parallel form, with its Q-flip pass and triangle reduction."""
    run_seq(oracle, 1, 520, 16, 2, 3, 3, 64, seed=72)
