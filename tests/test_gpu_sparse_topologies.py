"""GPU parity of the non-sequence sparse path (spiky_amd/csrc/lut_sparse.hip
behind spiky_lut_forward_step / spiky_lut_backward_backprop on a sparse
manager) over connectivity built directly, against the CPU oracle
(oracle/lut_oracle.c, restating lut_runtime_kernels_logic.proto:1160-1212,
1303-1545):

  * a ragged topology (every lookup neuron its own random target list): the
    atomic forward (fp32 sums in another order: |gpu - s| <= (n + 2) 2^-24 a,
    s the reference's sum, a the sum of the terms' magnitudes, n the most
    terms one output receives), the per-item propagate and the per-synapse
    weight gradient (bit-exact);
  * a uniform topology (the neurons of a detector share one target list) at
    batches that take the sample-lane forward, the row-slot propagate and the
    four-row weight-gradient walk: forward and weight gradient bit-exact.
"""
import numpy as np
import pytest
import torch

from spiky_amd import LUTDataManagerF

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def make_dm(I, O, T, Nc, fgs, off, tg):
    dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, fgs, 32)
    dm.register_synapse_meta(1.0, -10.0, 10.0, 0.0, 0.0)
    dm.initialize_neurons(False)
    dm.set_lookup_connectivity(off, tg)
    dm.compile(True, torch.zeros(tg.size))
    dm.to_device(0)
    return dm


def ragged_csr(rng, T, E, O, max_len):
    counts = rng.integers(0, max_len + 1, size=T * E)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    return off, rng.integers(0, O, size=int(off[-1])).astype(np.int32)


def uniform_csr(rng, T, E, O, max_len):
    rows = [rng.choice(O, size=int(rng.integers(1, max_len + 1)), replace=False).astype(np.int32)
            for _ in range(T)]
    tg = np.concatenate([np.tile(r, E) for r in rows])
    off = np.concatenate([[0], np.cumsum(np.repeat([len(r) for r in rows], E))]).astype(np.int64)
    return off, tg


def run(oracle, B, I, T, Nc, O, fgs, max_len, uniform, seed):
    dev = torch.device("cuda:0")
    print(f"[sparse topo] B={B} I={I} T={T} Nc={Nc} O={O} fgs={fgs} uniform={uniform}", flush=True)
    rng = np.random.default_rng(seed)
    E = 1 << Nc
    off, tg = (uniform_csr if uniform else ragged_csr)(rng, T, E, O, max_len)
    max_groups = int((np.diff(off).max() + fgs - 1) // fgs)
    dm = make_dm(I, O, T, Nc, fgs, off, tg)
    W = rng.standard_normal(tg.size).astype(np.float32) * 0.05
    x = rng.standard_normal(B * I).astype(np.float32)
    anchors = np.stack([rng.choice(I, 2, replace=False) for _ in range(T * Nc)]).astype(np.int32).reshape(-1)
    g = rng.standard_normal(B * O).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    Wd, xd, ad, gd = t(W), t(x), t(anchors), t(g)
    out = torch.zeros(B * O, device=dev)
    li = torch.zeros(B * T, dtype=torch.int32, device=dev)
    md = torch.zeros(B * T, device=dev)
    mi = torch.zeros(B * T, dtype=torch.int32, device=dev)
    dm.forward_step(Wd, B, xd, ad, out, li, 0.0, w_min_anchor_deltas=md, w_min_anchor_delta_indices=mi)
    xg = torch.zeros(B * I, device=dev)
    wg = torch.empty(tg.size, device=dev)
    dm.backward_backprop(Wd, B, gd, ad, li, md, mi, xg, -1.0, wg, overwrite_weights_gradients=True)
    torch.cuda.synchronize()

    ridx, rmd, rmi = oracle.check_detectors(x, anchors, B, I, T, Nc)
    assert np.array_equal(li.cpu().numpy(), ridx)
    rout = oracle.fill_outputs_sparse(W, ridx, off, tg, B, O, T, E)
    got = out.cpu().numpy()
    if uniform:
        assert np.array_equal(got, rout)
    else:
        rabs = oracle.fill_outputs_sparse(np.abs(W), ridx, off, tg, B, O, T, E).astype(np.float64)
        n = int(np.bincount(tg, minlength=O).max())
        assert np.all(np.abs(got.astype(np.float64) - rout) <= (n + 2) * U * rabs)
    rxg = oracle.propagate_sparse(W, g, ridx, rmd, rmi, anchors, off, tg, B, I, O, T, Nc, E, fgs, max_groups)
    gx = xg.cpu().numpy().reshape(B, I)
    cx = rxg.reshape(B, I)
    scale = np.abs(cx).max(axis=1, keepdims=True) + 1e-30
    assert np.all(np.abs(gx - cx) <= 1e-5 * scale)
    rwg = np.zeros(tg.size, np.float32)
    oracle.gather_wgrad_sparse(g, ridx, off, tg, rwg, B, O, T, E)
    assert np.array_equal(wg.cpu().numpy(), rwg)


@pytest.mark.parametrize("B", [5, 70])
def test_sparse_ragged_topology(oracle, cuda_device, B):
    run(oracle, B, 48, 24, 4, 40, 8, 19, False, seed=B)


@pytest.mark.parametrize("B,fgs", [(50, 32), (100, 8), (129, 16)])
def test_sparse_uniform_topology(oracle, cuda_device, B, fgs):
    # rows of 1..40 entries: several forward groups at fgs 8 and 16
    run(oracle, B, 64, 40, 5, 96, fgs, 40, True, seed=B + fgs)
