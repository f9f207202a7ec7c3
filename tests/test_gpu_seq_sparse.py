"""GPU parity of sequence-concat mode over sparse lookup connectivity
(spiky_amd/csrc/lut_seq_sparse.hip behind spiky_lut_forward_step_concat /
spiky_lut_backward_backprop_concat on a sparse manager) against the CPU
oracle (oracle/lut_oracle.c, restating lut_runtime_kernels_logic.proto:
1906-2015, 3371-3627, 3837-3942).

Bars:
  * lookup indices and margins (tokens and positions): bit-exact;
  * int32 summation: every accumulator bit-exact (order-free payload sums);
  * fp32 outputs, input / positional and weight gradients: the same terms
    as the reference summed in another order, |gpu - s| <= (n + 2) 2^-24 a
    (+ n 1e-17 for the sub-EPS input pushes), where s is the terms' fp64 sum,
    a the sum of their magnitudes and n the most terms one element receives;
    with integer weights and gradients every sum is exact and compared bitwise.
"""
import numpy as np
import pytest
import torch

from spiky_amd import LUTDataManagerF, LUTDataManagerI

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def random_csr(rng, n_lookup, O, max_len):
    counts = rng.integers(0, max_len + 1, size=n_lookup)
    counts[rng.integers(0, n_lookup)] = max_len  # at least one full neuron
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    tg = rng.integers(0, O, size=int(off[-1])).astype(np.int32)
    return off, tg


def make_dm(I, O, T, Nc, S, Npe, fgs, off, tg, int_rescaler=None, lr=1.0):
    args = (I, O, T, Nc, S, Npe, 0, fgs, 32)
    dm = LUTDataManagerF(*args) if int_rescaler is None else LUTDataManagerI(*args, int_rescaler)
    dm.register_synapse_meta(lr, -10.0, 10.0, 0.0, 0.0)
    dm.initialize_neurons(False)
    dm.set_lookup_connectivity(off, tg)
    dm.compile(True, torch.zeros(tg.size))
    dm.to_device(0)
    return dm


def run(oracle, B, S, I, T, Nc, Npe, O, fgs, seed, int_rescaler=None, int_values=False, internal=False,
        lr=1.0, ext_lr=0.25):
    dev = torch.device("cuda:0")
    int_mode = int_rescaler is not None
    print(f"[seq sparse] B={B} S={S} I={I} T={T} Nc={Nc} Npe={Npe} O={O} fgs={fgs} int={int_mode} "
          f"int_values={int_values} internal={internal}", flush=True)
    rng = np.random.default_rng(seed)
    E = 1 << (2 * Nc + Npe)
    off, tg = random_csr(rng, T * E, O, 2 * fgs + 1)
    n_syn = tg.size
    max_groups = int((np.diff(off).max() + fgs - 1) // fgs)
    x = rng.standard_normal(B * S * I).astype(np.float32)
    anchors = np.stack([rng.choice(I, 2, replace=False) for _ in range(T * Nc)]).astype(np.int32).reshape(-1)
    pe = rng.uniform(-1, 1, (S - 1) * T * Npe).astype(np.float32)
    if int_values:
        W = rng.integers(-6, 7, size=n_syn).astype(np.float32)
        g = rng.integers(-3, 4, size=B * S * O).astype(np.float32)
    else:
        W = (rng.standard_normal(n_syn) * 0.1).astype(np.float32)
        g = rng.standard_normal(B * S * O).astype(np.float32)
    dm = make_dm(I, O, T, Nc, S, Npe, fgs, off, tg, int_rescaler, lr)
    assert dm.get_max_forward_groups_per_neuron() == max_groups
    Wd, xd, ad, gd = (torch.from_numpy(v).to(dev) for v in (W, x, anchors, g))
    ped = torch.from_numpy(pe).to(dev) if Npe else None
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
        dm.backward_backprop_concat(Wd, B, gd, ad, idx, md, mi, xg, ext_lr, pli, pmd, pmi, peg, None)
        wg = None
    else:
        wg = torch.empty_like(Wd)
        dm.backward_backprop_concat(Wd, B, gd, ad, idx, md, mi, xg, -1.0, pli, pmd, pmi, peg, wg,
                                    overwrite_weights_gradients=True)
    torch.cuda.synchronize()

    ridx, rmd, rmi = oracle.check_detectors(x, anchors, B * S, I, T, Nc)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(md.cpu().numpy(), rmd)
    assert np.array_equal(mi.cpu().numpy(), rmi)
    rpli = rpmd = rpmi = None
    if Npe:
        rpli, rpmd, rpmi = oracle.check_pe(pe, S, T, Npe)
        assert np.array_equal(pli.cpu().numpy(), rpli)
        assert np.array_equal(pmd.cpu().numpy(), rpmd)
        assert np.array_equal(pmi.cpu().numpy(), rpmi)
    geo = (B, S, O, T, Nc, Npe, fgs, max_groups)
    R = int_rescaler or 1.0
    eff = dict(lr=lr, external_lr=ext_lr if internal else -1.0)
    if int_mode:
        rout = oracle.fill_outputs_seq_sparse(W, ridx, rpli, off, tg, *geo, int_mode=True, int_rescaler=R)
        rxg, rpeg = oracle.propagate_seq_sparse(W, g, ridx, rmd, rmi, rpli, rpmd, rpmi, anchors, off, tg, B, I,
                                                O, T, S, Nc, Npe, fgs, max_groups, int_mode=True, int_rescaler=R)
        rwg = oracle.gather_wgrad_seq_sparse(g, ridx, rpli, off, tg, *geo, **eff, int_mode=True, int_rescaler=R)
        for buf in (rout, rxg, rpeg, rwg):
            if buf is not None:
                oracle.convert_int_to_float(buf, R)
        assert np.array_equal(out.cpu().numpy(), rout)
        assert np.array_equal(xg.cpu().numpy(), rxg)
        if Npe:
            assert np.array_equal(peg.cpu().numpy(), rpeg)
        assert np.array_equal(wg.cpu().numpy(), rwg)
        return
    n_fwd = T * S * max_groups * (2 * fgs + 1)
    rout = oracle.fill_outputs_seq_sparse(W, ridx, rpli, off, tg, *geo).astype(np.float64)
    rabs = oracle.fill_outputs_seq_sparse(np.abs(W), ridx, rpli, off, tg, *geo).astype(np.float64)
    got = out.cpu().numpy().astype(np.float64)
    if int_values:
        assert np.array_equal(got, rout)
    else:
        assert np.all(np.abs(got - rout) <= 2 * (n_fwd + 2) * U * rabs)
    _, _, (xs, xa), pb = oracle.propagate_seq_sparse(W, g, ridx, rmd, rmi, rpli, rpmd, rpmi, anchors, off, tg,
                                                     B, I, O, T, S, Nc, Npe, fgs, max_groups, bounds=True)
    n_x = 2 * T * S * max_groups
    err = np.abs(xg.cpu().numpy().astype(np.float64) - xs)
    assert np.all(err <= (n_x + 2) * U * xa + n_x * 1e-17), f"x_grad excess {np.max(err - (n_x + 2) * U * xa)}"
    assert xa.max() > 0
    if Npe:
        ps, pa = pb
        n_p = B * S * max_groups
        assert np.all(np.abs(peg.cpu().numpy().astype(np.float64) - ps) <= (n_p + 2) * U * pa)
    wsum = oracle.gather_wgrad_seq_sparse(g, ridx, rpli, off, tg, *geo, **eff).astype(np.float64)
    wabs = oracle.gather_wgrad_seq_sparse(np.abs(g), ridx, rpli, off, tg, *geo, lr=abs(eff["lr"] * (
        -eff["external_lr"] if internal else 1.0))).astype(np.float64)
    n_w = B * S * (S - 1) // 2
    if internal:
        want = W.astype(np.float64) + wsum
        got_w = Wd.cpu().numpy().astype(np.float64)
        assert np.all(np.abs(got_w - want) <= 2 * (n_w + 2) * U * (wabs + np.abs(W)))
    else:
        got_w = wg.cpu().numpy().astype(np.float64)
        if int_values:
            assert np.array_equal(got_w, wsum)
        else:
            assert np.all(np.abs(got_w - wsum) <= 2 * (n_w + 2) * U * wabs)


@pytest.mark.parametrize("Npe", [0, 2])
def test_seq_sparse_fp32(oracle, cuda_device, Npe):
    run(oracle, B=2, S=9, I=12, T=3, Nc=2, Npe=Npe, O=10, fgs=3, seed=1)


def test_seq_sparse_integer_values_exact(oracle, cuda_device):
    run(oracle, B=2, S=11, I=10, T=2, Nc=3, Npe=1, O=9, fgs=4, seed=2, int_values=True)


@pytest.mark.parametrize("Npe", [0, 2])
def test_seq_sparse_int32_bit_exact(oracle, cuda_device, Npe):
    run(oracle, B=2, S=8, I=12, T=3, Nc=2, Npe=Npe, O=10, fgs=3, seed=3, int_rescaler=0.001)


def test_seq_sparse_internal_policy(oracle, cuda_device):
    """Internal SGD: the weights move after the input gradient read them."""
    run(oracle, B=2, S=7, I=10, T=2, Nc=2, Npe=1, O=8, fgs=2, seed=4, internal=True, lr=0.5)


def test_seq_sparse_longer_than_a_tile(oracle, cuda_device):
    """S = 40 crosses the reference's 32-wide pair tiles."""
    run(oracle, B=1, S=40, I=8, T=2, Nc=2, Npe=1, O=6, fgs=3, seed=5)


def test_seq_sparse_conv2d_layer_autograd(oracle, cuda_device):
    """A Conv2DLUTLayer attention with a lookup receptive field (the reference's
    sparse sequence topology, LUTLayer.py:1285-1380) through autograd."""
    from spiky_amd.lut.LUTLayer import Conv2DLUTLayer, SynapseMeta
    dev = cuda_device
    S = 6
    layer = Conv2DLUTLayer(input_shape=(4, 4), n_anchors_per_detector=2, detectors_shape=(2, 2),
                           output_kernel_shape=(2, 2), sequence_length=S, receptive_field_shape=(2, 2),
                           receptive_field_stride_shape=(1, 1), lut_receptive_field_shape=(4, 4),
                           lut_receptive_field_stride_shape=(2, 2), positional_dim=0,
                           synapse_meta=SynapseMeta(initial_noise_level=1.0), _forward_group_size=3,
                           random_seed=3, device=dev)
    off, tg = layer._lut_dm.lookup_connectivity()
    T, Nc, O = layer.n_detectors(), layer.n_anchors_per_detector(), layer.n_outputs()
    I = 16
    fgs = 3
    max_groups = layer._lut_dm.get_max_forward_groups_per_neuron()
    g = torch.Generator().manual_seed(4)
    B = 3
    x = torch.randn(B, S, 4, 4, generator=g).to(dev).requires_grad_(True)
    y = layer(x)
    go = torch.randn(B, S, 4, 4, generator=g).to(dev)
    y.backward(go)
    torch.cuda.synchronize()
    xn = x.detach().cpu().numpy().reshape(-1)
    anchors = layer._detector_anchors.cpu().numpy()
    W = layer._weights.detach().cpu().numpy()
    ridx, rmd, rmi = oracle.check_detectors(xn, anchors, B * S, I, T, Nc)
    geo = (B, S, O, T, Nc, 0, fgs, max_groups)
    rout = oracle.fill_outputs_seq_sparse(W, ridx, None, off, tg, *geo).astype(np.float64)
    rabs = oracle.fill_outputs_seq_sparse(np.abs(W), ridx, None, off, tg, *geo).astype(np.float64)
    n_fwd = T * S * max_groups * fgs
    assert np.all(np.abs(y.detach().cpu().numpy().reshape(-1) - rout) <= 2 * (n_fwd + 2) * U * rabs)
    gn = go.cpu().numpy().reshape(-1)
    _, _, (xs, xa), _ = oracle.propagate_seq_sparse(W, gn, ridx, rmd, rmi, None, None, None, anchors, off, tg,
                                                    B, I, O, T, S, Nc, 0, fgs, max_groups, bounds=True)
    n_x = 2 * T * S * max_groups
    assert np.all(np.abs(x.grad.cpu().numpy().reshape(-1) - xs) <= (n_x + 2) * U * xa + n_x * 1e-17)
    wsum = oracle.gather_wgrad_seq_sparse(gn, ridx, None, off, tg, *geo).astype(np.float64)
    wabs = oracle.gather_wgrad_seq_sparse(np.abs(gn), ridx, None, off, tg, *geo).astype(np.float64)
    n_w = B * S * (S - 1) // 2
    assert np.all(np.abs(layer._weights.grad.cpu().numpy() - wsum) <= 2 * (n_w + 2) * U * wabs)
    assert np.abs(wsum).max() > 0
