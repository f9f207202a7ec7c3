"""GPU parity of the fully connected LUT path against the CPU oracle.

Bars (fixed by the task's north star):
  * lookup indices, min-margin values and indices: bit-exact;
  * forward output: bit-exact (the kernel keeps the reference CPU path's block
    grouping and commit order);
  * weight gradient: bit-exact (table-major bucketed kernel, ascending samples);
  * int32 summation (forward, input and weight gradients): bit-exact;
  * fp32 input gradient: the reference commits it with atomics, so only a
    tolerance applies: |gpu - cpu| <= 1e-5 * max|x_grad[b, :]| per sample row.
"""
import numpy as np
import pytest
import torch

from spiky_amd import LUTDataManagerF, LUTDataManagerI

pytestmark = pytest.mark.gpu

XG_RTOL = 1e-5


def make_dm(I, O, T, Nc, fgs=32, bgs=32, int_rescaler=None, lr=1.0):
    if int_rescaler is None:
        dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, fgs, bgs)
    else:
        dm = LUTDataManagerI(I, O, T, Nc, 1, 0, 0, fgs, bgs, int_rescaler)
    dm.register_synapse_meta(lr, -10.0, 10.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    return dm


def make_inputs(seed, B, I, T, Nc, O, x_normal=False):
    g = torch.Generator().manual_seed(seed)
    E = 1 << Nc
    x = torch.randn(B * I, generator=g) if x_normal else torch.rand(B * I, generator=g)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    W = torch.randn(T * E * O, generator=g) * 0.01
    go = torch.randn(B * O, generator=g)
    return x, anchors, W, go


def xg_close(gpu, cpu, B, I, T=8192, n_ob=32, extra=0.0):
    """|gpu - cpu| <= 1e-5 * max|x_grad[b, :]| + T * n_ob * 1e-17.  The absolute
    term bounds the terms the reference drops as |du| <= EPS = 1e-17 per
    (table, 32-output block) (misc.h:90, proto:833-863) where a kernel that
    commits wider sums applies the same cut to the sum instead."""
    gpu = gpu.reshape(B, I)
    cpu = cpu.reshape(B, I)
    scale = np.abs(cpu).max(axis=1, keepdims=True)
    err = np.abs(gpu - cpu)
    bound = XG_RTOL * scale + T * n_ob * 1e-17 + extra
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"


def run_fc(oracle, B, I, T, Nc, O, fgs=32, bgs=32, cmp_eps=0.0, seed=0, int_rescaler=None, lr=1.0,
           edit_grad=None, wg_exact=True, edit_anchors=None, xg_extra=0.0):
    dev = torch.device("cuda:0")
    E = 1 << Nc
    int_mode = int_rescaler is not None
    x, anchors, W, go = make_inputs(seed, B, I, T, Nc, O)
    if edit_grad is not None:
        go = edit_grad(go)
    if edit_anchors is not None:
        anchors = edit_anchors(anchors)
    dm = make_dm(I, O, T, Nc, fgs, bgs, int_rescaler, lr)
    xd, ad, Wd, gd = x.to(dev), anchors.to(dev), W.to(dev), go.to(dev)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    md = torch.empty(B * T, device=dev)
    mi = torch.empty(B * T, dtype=torch.int32, device=dev)
    print(f"[fc] B={B} I={I} T={T} Nc={Nc} O={O} fgs={fgs} bgs={bgs} int={int_mode}", flush=True)
    dm.forward_step(Wd, B, xd, ad, out, idx, cmp_eps, None, md, mi)
    xg = torch.zeros(B * I, device=dev)
    wg = torch.empty(T * E * O, device=dev)
    dm.backward_backprop(Wd, B, gd, ad, idx, md, mi, xg, -1.0, wg, None,
                         overwrite_weights_gradients=True)
    wg_acc = torch.zeros(T * E * O, device=dev)
    xg2 = torch.zeros(B * I, device=dev)
    dm.backward_backprop(Wd, B, gd, ad, idx, md, mi, xg2, -1.0, wg_acc, None)
    torch.cuda.synchronize()
    # oracle
    xn, an, Wn, gn = x.numpy(), anchors.numpy(), W.numpy(), go.numpy()
    ridx, rmd, rmi = oracle.check_detectors(xn, an, B, I, T, Nc, cmp_eps)
    rout = oracle.fill_outputs_fc(Wn, ridx, B, O, T, E, dgs=bgs, int_mode=int_mode,
                                  int_rescaler=int_rescaler or 1.0)
    if int_mode:
        oracle.convert_int_to_float(rout, int_rescaler)
    rxg = oracle.propagate_fc(Wn, gn, ridx, rmd, rmi, an, B, I, O, T, Nc, E, ogs=fgs,
                              int_mode=int_mode, int_rescaler=int_rescaler or 1.0)
    if int_mode:
        oracle.convert_int_to_float(rxg, int_rescaler)
    rwg = np.zeros(T * E * O, np.float32)
    oracle.gather_wgrad_fc(gn, ridx, rwg, B, O, T, E, ogs=fgs, first_meta_lr=lr, int_mode=int_mode,
                           int_rescaler=int_rescaler or 1.0)
    if int_mode:
        oracle.convert_int_to_float(rwg, int_rescaler)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(md.cpu().numpy(), rmd)
    assert np.array_equal(mi.cpu().numpy(), rmi)
    assert np.array_equal(out.cpu().numpy(), rout)
    n_ob = (O + fgs - 1) // fgs
    if int_mode:
        assert np.array_equal(xg.cpu().numpy(), rxg)
        assert np.array_equal(xg2.cpu().numpy(), rxg)
    else:
        xg_close(xg.cpu().numpy(), rxg, B, I, T, n_ob, xg_extra)
        xg_close(xg2.cpu().numpy(), rxg, B, I, T, n_ob, xg_extra)
    if wg_exact:
        assert np.array_equal(wg.cpu().numpy(), rwg)
        assert np.array_equal(wg_acc.cpu().numpy(), rwg)
    else:
        # fp32 sums committed with atomics in any order: within B * 2^-24 of
        # the sum of the terms' magnitudes (the oracle's own sum of |g * lr|)
        rabs = np.zeros(T * E * O, np.float32)
        oracle.gather_wgrad_fc(np.abs(gn), ridx, rabs, B, O, T, E, ogs=fgs, first_meta_lr=lr)
        bound = B * 2.0 ** -24 * rabs.astype(np.float64) * 1.01
        for got in (wg, wg_acc):
            err = np.abs(got.cpu().numpy().astype(np.float64) - rwg)
            assert np.all(err <= bound), f"max excess {np.max(err - bound)}"


def test_config1_full(oracle, cuda_device):
    run_fc(oracle, 64, 784, 256, 6, 10)


def test_config3_shrunk(oracle, cuda_device):
    run_fc(oracle, 16, 512, 256, 8, 1024, seed=1)


def test_large_batch_ragged_slices(oracle, cuda_device):
    # 4 samples per wavefront with a ragged last wavefront; 16 column slices, the
    # last one partly inactive (1000 = 15*64 + 40)
    run_fc(oracle, 515, 256, 40, 5, 1000, seed=11)


def test_large_batch_two_columns_per_lane(oracle, cuda_device):
    # 2 columns per lane; block sizes that do not divide the table count or the unroll
    run_fc(oracle, 600, 128, 24, 4, 1024, fgs=16, bgs=7, seed=12)


def test_large_batch_four_columns_per_lane(oracle, cuda_device):
    run_fc(oracle, 520, 96, 16, 3, 2048, seed=13)


def test_table_major_two_sample_chunks(oracle, cuda_device):
    # 256-entry tables staged in LDS, a second sample chunk of 6 samples, and a
    # last column slice of 4 columns (100 = 3*32 + 4)
    run_fc(oracle, 1030, 300, 40, 8, 100, seed=15)


@pytest.mark.parametrize("B,O", [(256, 128), (300, 192), (1100, 64)])
def test_table_major_wide_slices(oracle, cuda_device, B, O):
    # 256-entry tables and O % 64 == 0: the propagate's 64-column slices (16
    # lanes per 256-byte row) with 4, 8 and 16 samples per lane, and a second
    # sample chunk of 76 samples
    run_fc(oracle, B, 300, 40, 8, O, seed=16)


@pytest.mark.parametrize("int_rescaler", [None, 0.5])
def test_table_major_dma_forward_two_chunks(oracle, cuda_device, int_rescaler):
    # 256-entry tables and more than 1024 samples: the LDS-DMA forward over two
    # sample chunks (the second of 76 samples) and two units of 32 and 8
    # tables, fp32 and int32 summation
    run_fc(oracle, 1100, 300, 40, 8, 128, seed=17, int_rescaler=int_rescaler)


def test_many_samples_few_tables(oracle, cuda_device):
    # 4100 samples over 6 tables: the weight gradient's bucket sort runs a
    # workgroup per table, with a ragged last 64-sample group
    run_fc(oracle, 4100, 64, 6, 4, 64, seed=19)


@pytest.mark.parametrize("T,B,O", [(192, 8192, 64), (64, 8192, 128)])
def test_few_tables_many_samples_unit_sizes(oracle, cuda_device, T, B, O):
    # few 256-entry tables over many samples, a transformer feed-forward layer's
    # shape: so that the grid still covers the CUs, the whole-table propagate
    # takes 4 (T 192) or 2 (T 64) tables a unit over 8 sample chunks, and the
    # weight gradient 8 or 4 rows a wavefront.  Every sum and its order are
    # unchanged, so the usual bars hold (1 table a unit is the config-5 test's)
    run_fc(oracle, B, 256, T, 8, O, seed=21)


def test_large_batch_int32_summation(oracle, cuda_device):
    run_fc(oracle, 530, 64, 20, 4, 512, seed=14, int_rescaler=0.5)


def test_weight_gradient_eps_edge(oracle, cuda_device):
    # gradient values on both sides of the reference's |g| > 1e-17 cut (misc.h:90),
    # through the lr == 1 fp32 path (O = 1024: four columns per lane)
    eps = np.float32(1e-17)
    edge = np.array([eps, -eps, np.nextafter(eps, np.float32(1)), np.nextafter(eps, np.float32(0)),
                     -np.nextafter(eps, np.float32(1)), 0.0, -0.0, 1e-30, 1e-16], np.float32)

    def edit(go):
        g = go.numpy().copy()
        g[: g.size // 2] = np.resize(edge, g.size // 2)
        return torch.from_numpy(g)

    run_fc(oracle, 40, 64, 24, 4, 1024, seed=16, edit_grad=edit)
    run_fc(oracle, 40, 64, 24, 4, 1024, seed=16, edit_grad=edit, lr=0.5)


def test_unusual_group_sizes(oracle, cuda_device):
    # the reference's own tests use odd block sizes (test_lut_transformer_small.py:287-291)
    run_fc(oracle, 7, 50, 70, 5, 37, fgs=4, bgs=24, seed=2)


def test_wide_outputs_and_eps(oracle, cuda_device):
    run_fc(oracle, 5, 64, 40, 3, 1536, seed=3, cmp_eps=0.05)


@pytest.mark.parametrize("Nc,int_rescaler", [(10, None), (10, 0.5), (13, None), (13, 0.5)])
def test_many_entries(oracle, cuda_device, Nc, int_rescaler):
    """Tables of 2^10 and 2^13 rows (16-pair anchor registers in the check, the
    per-sample forward).  Up to 4096 rows the weight gradient is the bucketed
    walk (bit-exact); past it, the atomic form, whose fp32 sums are order-free
    as the reference GPU path's are (int32 sums stay bit-exact)."""
    run_fc(oracle, 70, 200, 6, Nc, 48, seed=31, int_rescaler=int_rescaler,
           wg_exact=Nc <= 12 or int_rescaler is not None)


@pytest.mark.parametrize("int_rescaler", [None, 0.5])
def test_degenerate_anchor_pairs(oracle, cuda_device, int_rescaler):
    """Explicit anchors need not be distinct: pairs drawn with repetition,
    every fourth pair comparing an input with itself (Δ = 0: bit 0, and its
    two input-gradient pushes cancel), several tables sharing inputs.  The
    large batch takes the table-major kernels, the small one the per-sample
    ones.  Such a pair is most tables' min-margin pair (|Δ| = 0), so each
    input takes up to 2T pushes of ±du (|du| <= 0.5) that cancel: int32 sums
    stay bit-exact, but an fp32 input gradient is then the rounding residue of
    that cancellation, set by the order of the pushes, which the reference's
    fp32 atomics leave free.  Its bar adds the order freedom of 2T fp32 adds
    whose partial sums stay within T * 0.5: 2T * T * 2^-24."""
    def edit(a):
        g = torch.Generator().manual_seed(41)
        a = torch.randint(0, 24, a.shape, generator=g, dtype=torch.int32)
        a = a.view(-1, 2)
        a[::4, 1] = a[::4, 0]
        return a.flatten().contiguous()
    for B in (9, 300):
        run_fc(oracle, B, 24, 40, 5, 64, seed=42, int_rescaler=int_rescaler, edit_anchors=edit,
               xg_extra=2 * 40 * 40 * 2.0 ** -24)


def test_check_without_lds_staging(oracle, cuda_device):
    """The detector check's other kernel: rows past 16384 inputs (no four-sample
    group fits the LDS) and tables past 16 pairs (2^17 rows; their weight
    gradient is the atomic form)."""
    run_fc(oracle, 5, 20000, 3, 4, 8, seed=61)
    run_fc(oracle, 6, 64, 2, 17, 4, seed=62, wg_exact=False)
    run_fc(oracle, 6, 64, 2, 17, 4, seed=63, int_rescaler=0.5)


@pytest.mark.parametrize("int_rescaler", [None, 0.5])
def test_large_batch_odd_outputs(oracle, cuda_device, int_rescaler):
    """A batch past 256 with 10 and 66 outputs (not whole 4-column pieces: the
    table-major kernels do not take it) and a batch of exactly 256 with 64."""
    run_fc(oracle, 300, 50, 30, 5, 10, seed=81, int_rescaler=int_rescaler)
    run_fc(oracle, 260, 50, 30, 5, 66, seed=82, int_rescaler=int_rescaler)
    run_fc(oracle, 256, 50, 30, 5, 64, seed=83, int_rescaler=int_rescaler)


def test_single_sample_single_table(oracle, cuda_device):
    run_fc(oracle, 1, 2, 1, 1, 1, seed=4)


def test_learning_rate(oracle, cuda_device):
    run_fc(oracle, 9, 32, 33, 4, 64, seed=5, lr=0.25)


def test_int32_summation(oracle, cuda_device):
    run_fc(oracle, 8, 64, 100, 4, 48, seed=6, int_rescaler=0.5)
    run_fc(oracle, 8, 64, 100, 4, 10, seed=7, int_rescaler=0.001)


def test_eval_mode(oracle, cuda_device):
    dev = cuda_device
    B, I, T, Nc, O = 6, 100, 64, 6, 96
    x, anchors, W, _ = make_inputs(8, B, I, T, Nc, O)
    dm = make_dm(I, O, T, Nc)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    dm.forward_step(W.to(dev), B, x.to(dev), anchors.to(dev), out, idx)
    ridx = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc, train=False)
    rout = oracle.fill_outputs_fc(W.numpy(), ridx, B, O, T, 1 << Nc)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(out.cpu().numpy(), rout)


def test_internal_policy_sgd(oracle, cuda_device):
    dev = cuda_device
    B, I, T, Nc, O = 5, 40, 50, 4, 64
    E = 1 << Nc
    x, anchors, W, go = make_inputs(9, B, I, T, Nc, O)
    dm = make_dm(I, O, T, Nc, lr=0.5)
    Wd = W.to(dev)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    md = torch.empty(B * T, device=dev)
    mi = torch.empty(B * T, dtype=torch.int32, device=dev)
    dm.forward_step(Wd, B, x.to(dev), anchors.to(dev), out, idx, 0.0, None, md, mi)
    xg = torch.zeros(B * I, device=dev)
    dm.backward_backprop(Wd, B, go.to(dev), anchors.to(dev), idx, md, mi, xg, 0.1, None)
    with pytest.raises(ValueError):
        dm.backward_backprop(Wd, B, go.to(dev), anchors.to(dev), idx, md, mi, xg, 0.1,
                             torch.zeros_like(Wd))
    ridx, rmd, rmi = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc)
    rxg = oracle.propagate_fc(W.numpy(), go.numpy(), ridx, rmd, rmi, anchors.numpy(), B, I, O, T,
                              Nc, E)
    rW = W.numpy().copy()
    oracle.gather_wgrad_fc(go.numpy(), ridx, rW, B, O, T, E, first_meta_lr=0.5,
                           external_lr=np.float32(0.1))
    xg_close(xg.cpu().numpy(), rxg, B, I, T, 2)
    assert np.array_equal(Wd.cpu().numpy(), rW)


@pytest.mark.parametrize("B,O", [(12, 128), (517, 1024), (300, 100), (300, 66)])
def test_int8_tables(oracle, cuda_device, B, O):
    dev = cuda_device
    I, T, Nc = 256, 96, 6
    E = 1 << Nc
    g = torch.Generator().manual_seed(10)
    x = torch.randn(B * I, generator=g)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    q = torch.randint(-127, 128, (T * E * O,), generator=g, dtype=torch.int8)
    sc = torch.rand(T, generator=g) * 0.009 + 0.001
    for resc in (None, 1.0):
        dm = make_dm(I, O, T, Nc, int_rescaler=resc)
        out = torch.zeros(B * O, device=dev)
        idx = torch.empty(B * T, dtype=torch.int32, device=dev)
        dm.forward_step_i8(q.to(dev), sc.to(dev), B, x.to(dev), anchors.to(dev), out, idx)
        ridx = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc, train=False)
        rout = oracle.fill_outputs_fc(None, ridx, B, O, T, E, q8=q.numpy(), scales=sc.numpy(),
                                      int_mode=resc is not None, int_rescaler=resc or 1.0)
        if resc is not None:
            oracle.convert_int_to_float(rout, resc)
        assert np.array_equal(idx.cpu().numpy(), ridx)
        assert np.array_equal(out.cpu().numpy(), rout)


@pytest.mark.parametrize("tables", ["int8", "fp32"])
def test_table_major_folded_blocks(oracle, cuda_device, tables):
    """int32 summation with many 8-table blocks: the table-major forward folds
    several blocks' payloads into one partial (wrapping int32 sums are
    associative); every accumulator must still be bit-exact."""
    dev = cuda_device
    B, I, T, Nc, O, dgs, resc = 300, 256, 16384, 6, 64, 8, 0.25
    E = 1 << Nc
    g = torch.Generator().manual_seed(31)
    x = torch.randn(B * I, generator=g)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    dm = make_dm(I, O, T, Nc, 32, dgs, int_rescaler=resc)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    if tables == "int8":
        q = torch.randint(-127, 128, (T * E * O,), generator=g, dtype=torch.int8)
        sc = torch.rand(T, generator=g) * 0.009 + 0.001
        dm.forward_step_i8(q.to(dev), sc.to(dev), B, x.to(dev), anchors.to(dev), out, idx)
        kw = dict(q8=q.numpy(), scales=sc.numpy())
        W = None
    else:
        W = (torch.randn(T * E * O, generator=g) * 0.01)
        dm.forward_step(W.to(dev), B, x.to(dev), anchors.to(dev), out, idx)
        kw = {}
        W = W.numpy()
    ridx = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc, train=False)
    rout = oracle.fill_outputs_fc(W, ridx, B, O, T, E, dgs=dgs, int_mode=True, int_rescaler=resc, **kw)
    oracle.convert_int_to_float(rout, resc)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(out.cpu().numpy(), rout)


@pytest.mark.parametrize("ordered", [False, True])
def test_forward_fold_modes(oracle, cuda_device, ordered):
    """Table-major fp32 forward with two 1024-sample chunks and 128 blocks of
    32 tables (2048 units): ordered sums give the reference CPU path's output
    bit for bit; the default folds two blocks into one fp64 sum, which is the
    oracle's arithmetic with 64-table blocks, bit for bit, and within 1e-5 of
    each row's largest output of the ordered result."""
    from test_gpu_layers import fold_blocks
    dev = cuda_device
    B, I, T, Nc, O = 2048, 300, 4096, 8, 256
    E = 1 << Nc
    x, anchors, W, _ = make_inputs(21, B, I, T, Nc, O, x_normal=True)
    dm = make_dm(I, O, T, Nc)
    dm.set_ordered_sums(ordered)
    fold = 1 if ordered else fold_blocks(B, T, O)
    assert ordered or fold == 2
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    print(f"[fold] ordered={ordered} fold={fold}", flush=True)
    dm.forward_step(W.to(dev), B, x.to(dev), anchors.to(dev), out, idx)
    torch.cuda.synchronize()
    ridx = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc, train=False)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    got = out.cpu().numpy()
    assert np.array_equal(got, oracle.fill_outputs_fc(W.numpy(), ridx, B, O, T, E, dgs=32 * fold))
    r32 = oracle.fill_outputs_fc(W.numpy(), ridx, B, O, T, E, dgs=32).reshape(B, O)
    assert np.all(np.abs(got.reshape(B, O) - r32) <= 1e-5 * np.abs(r32).max(axis=1, keepdims=True))


def test_errors_on_device(cuda_device):
    dev = cuda_device
    dm = make_dm(8, 4, 4, 2)
    W = torch.zeros(4 * 4 * 4, device=dev)
    with pytest.raises(ValueError, match="no active context"):
        dm.backward_backprop(W, 1, torch.zeros(4, device=dev), torch.zeros(16, dtype=torch.int32, device=dev),
                             torch.zeros(4, dtype=torch.int32, device=dev), torch.zeros(4, device=dev),
                             torch.zeros(4, dtype=torch.int32, device=dev), torch.zeros(8, device=dev), -1.0)
    with pytest.raises(RuntimeError, match="must be on CUDA"):
        dm.forward_step(W.cpu(), 1, torch.zeros(8, device=dev), torch.zeros(16, dtype=torch.int32, device=dev),
                        torch.zeros(4, device=dev), torch.zeros(4, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError, match="batch_size == 0"):
        dm.forward_step(W, 0, torch.zeros(8, device=dev), torch.zeros(16, dtype=torch.int32, device=dev),
                        torch.zeros(4, device=dev), torch.zeros(4, dtype=torch.int32, device=dev))


def test_forward_batch_dependence(cuda_device):
    """The fold of the default fp32 forward is chosen from the shape and the
    batch (enough blocks to leave about 1024 work units), so the same sample's
    output bits can differ between batch sizes: here 8 blocks a partial at
    B = 4096 and 2 at B = 1024, and the ordered 32-table commits of the
    small-batch kernel at B = 200.  Every pair stays within 1e-5 of the row's
    largest output; with ordered sums the three are bit-identical."""
    from test_gpu_layers import fold_blocks
    dev = cuda_device
    I, T, Nc, O = 128, 8192, 8, 256
    assert (fold_blocks(4096, T, O), fold_blocks(1024, T, O)) == (8, 2)
    x, anchors, W, _ = make_inputs(23, 4096, I, T, Nc, O, x_normal=True)
    Wd, xd, ad = W.to(dev), x.to(dev), anchors.to(dev)
    outs = {}
    for ordered in (False, True):
        dm = make_dm(I, O, T, Nc)
        dm.set_ordered_sums(ordered)
        for B in (4096, 1024, 200):
            print(f"[batch dependence] ordered={ordered} B={B}", flush=True)
            out = torch.zeros(B * O, device=dev)
            idx = torch.empty(B * T, dtype=torch.int32, device=dev)
            dm.forward_step(Wd, B, xd[:B * I], ad, out, idx)
            torch.cuda.synchronize()
            outs[ordered, B] = out.view(B, O)[:200].cpu()
    for ordered in (False, True):
        a, b, c = (outs[ordered, B] for B in (4096, 1024, 200))
        if ordered:
            assert torch.equal(a.view(torch.int32), c.view(torch.int32))
            assert torch.equal(b.view(torch.int32), c.view(torch.int32))
        else:
            scale = c.abs().max(dim=1, keepdim=True).values
            for got in (a, b):
                assert torch.all((got - c).abs() <= 1e-5 * scale)
            assert not torch.equal(a, c), "the folded forward is expected to round differently somewhere"
    assert torch.equal(outs[True, 200], outs[False, 200])
