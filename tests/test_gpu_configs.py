"""GPU parity at the benchmark configurations that have their own kernel
instantiations: config 4 (int8 tables, int32 summation, E = 256 rows, folded
int32 blocks over several 1024-sample chunks) and config 2 (the sparse
ProjectionLUTLayer stack plus its dense head), and NaN inputs through the
detector check.

Bars: lookup indices, min-margin values and indices, forward outputs, int32
accumulators and weight gradients bit-exact; fp32 input gradients within
1e-5 of each sample row's largest magnitude (the reference adds them with
fp32 atomics in any order)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _xg_close(gpu, cpu, B, I, rtol=1e-5, abs_eps=0.0):
    gpu = np.asarray(gpu).reshape(B, I)
    cpu = np.asarray(cpu).reshape(B, I)
    bound = rtol * np.abs(cpu).max(axis=1, keepdims=True) + abs_eps
    err = np.abs(gpu - cpu)
    assert np.all(err <= bound), f"max excess {np.max(err - bound)}"


def _int8_manager(I, O, T, Nc, dgs, resc):
    from spiky_amd import LUTDataManagerI
    dm = LUTDataManagerI(I, O, T, Nc, 1, 0, 0, 32, dgs, resc)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    return dm


def test_config4_full_shape(oracle, cuda_device):
    """BASELINE config 4 as the bench runs it: 8192 int8 tables of 256 rows x
    1024 outputs (2.1 GB), per-table scales in [0.001, 0.01], int_rescaler
    0.001, 32-table blocks, batch 4096 (four 1024-sample chunks, 16 blocks
    folded per unit).  A sample's output depends only on its own 8192 rows, so
    each checked sample's rows are gathered host-side into an E = 1 table and
    run through the oracle's int8 path (proto:1276-1285 payloads,
    proto:200-213 epilogue): bit-exact."""
    dev = cuda_device
    B, I, T, Nc, O, resc = 4096, 4096, 8192, 8, 1024, 0.001
    E = 1 << Nc
    gq = torch.Generator(device=dev).manual_seed(4)
    q8 = torch.randint(-127, 128, (T * E * O,), device=dev, generator=gq, dtype=torch.int8)
    sc = torch.rand(T, device=dev, generator=gq) * 0.009 + 0.001
    x = torch.randn(B * I, device=dev, generator=gq)
    ga = torch.Generator().manual_seed(1)
    anchors = torch.stack([torch.randperm(I, generator=ga)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    dm = _int8_manager(I, O, T, Nc, 32, resc)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    print("[config4] forward_step_i8 B=4096 T=8192 Nc=8 O=1024", flush=True)
    dm.forward_step_i8(q8, sc, B, x, anchors.to(dev), out, idx)
    torch.cuda.synchronize()
    samples = [0, 1023, 1024, 2047, 2900, B - 1]
    xs = x.view(B, I)[samples].cpu().numpy().reshape(-1)
    ridx = oracle.check_detectors(xs, anchors.numpy(), len(samples), I, T, Nc, train=False)
    assert np.array_equal(idx.view(B, T)[samples].cpu().numpy().reshape(-1), ridx)
    qv = q8.view(T, E, O)
    tt = torch.arange(T, device=dev)
    scn = sc.cpu().numpy()
    for s in samples:
        rows = qv[tt, idx.view(B, T)[s].long()].cpu().numpy().reshape(-1)    # [T][O], E = 1
        r = oracle.fill_outputs_fc(None, np.zeros((1, T), np.int32), 1, O, T, 1, dgs=32, q8=rows,
                                   scales=scn, int_mode=True, int_rescaler=resc)
        oracle.convert_int_to_float(r, resc)
        assert np.array_equal(out.view(B, O)[s].cpu().numpy(), r), f"sample {s}"


@pytest.mark.parametrize("B,dgs", [(2100, 8), (1300, 32)])
def test_int8_e256_chunks_and_folds(oracle, cuda_device, B, dgs):
    """The int8 table-major forward at E = 256 (one LDS row per entry) with
    ragged batches over two and three 1024-sample chunks; with 8-table blocks
    several blocks are folded into one int32 partial.  The whole output is
    compared with the oracle, bit for bit."""
    dev = cuda_device
    I, T, Nc, O, resc = 512, 2048, 8, 256, 0.001
    E = 1 << Nc
    g = torch.Generator().manual_seed(40 + dgs)
    x = torch.randn(B * I, generator=g)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    q = torch.randint(-127, 128, (T * E * O,), generator=g, dtype=torch.int8)
    sc = torch.rand(T, generator=g) * 0.009 + 0.001
    dm = _int8_manager(I, O, T, Nc, dgs, resc)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    print(f"[int8 e256] B={B} dgs={dgs}", flush=True)
    dm.forward_step_i8(q.to(dev), sc.to(dev), B, x.to(dev), anchors.to(dev), out, idx)
    torch.cuda.synchronize()
    ridx = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc, train=False)
    rout = oracle.fill_outputs_fc(None, ridx, B, O, T, E, dgs=dgs, q8=q.numpy(), scales=sc.numpy(),
                                  int_mode=True, int_rescaler=resc)
    oracle.convert_int_to_float(rout, resc)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(out.cpu().numpy(), rout)



@pytest.mark.parametrize("ordered", [True, False])
def test_int8_e256_fp32_sums_partial_slice(oracle, cuda_device, ordered):
    """int8 tables at E = 256 with fp32 summation (LUTDataManagerF): two
    ragged 1024-sample chunks and 112 outputs, so the last 32-column slice is
    half past the row (its loads clamp, its stores are skipped).  Ordered sums
    commit every 32-table block in order, as the reference; folded ones form
    one fp64 sum over the unit's blocks, which is the oracle with blocks of
    that many tables.  Bit for bit either way."""
    from test_gpu_layers import fold_blocks
    from spiky_amd import LUTDataManagerF
    dev = cuda_device
    B, I, T, Nc, O = 1500, 300, 8192, 8, 112
    E = 1 << Nc
    g = torch.Generator().manual_seed(77)
    x = torch.randn(B * I, generator=g)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    q = torch.randint(-128, 128, (T * E * O,), generator=g, dtype=torch.int8)
    sc = torch.rand(T, generator=g) * 0.009 + 0.001
    dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, 32, 32)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    dm.set_ordered_sums(ordered)
    fold = 1 if ordered else fold_blocks(B, T, O)
    assert ordered or fold == 2
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    print(f"[int8 fp32 sums] ordered={ordered} fold={fold}", flush=True)
    dm.forward_step_i8(q.to(dev), sc.to(dev), B, x.to(dev), anchors.to(dev), out, idx)
    torch.cuda.synchronize()
    ridx = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc, train=False)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    rout = oracle.fill_outputs_fc(None, ridx, B, O, T, E, dgs=32 * fold, q8=q.numpy(), scales=sc.numpy())
    assert np.array_equal(out.cpu().numpy(), rout)


def test_config2_projection_stack(oracle, cuda_device):
    """BASELINE config 2 as the bench builds it (bench.build_projection_stack):
    two sparse ProjectionLUTLayers and the 800 -> 10 dense head at batch 128,
    forward and backward through autograd.  Each layer is checked against the
    oracle on the inputs and upstream gradients the GPU chain gave it: outputs
    and weight gradients bit-exact, input gradients within the row bound."""
    from bench import build_projection_stack
    dev = cuda_device
    B = 128
    l1, l2, head = build_projection_stack(dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    with torch.no_grad():
        for layer in (l1, l2, head):
            layer._weights.normal_(0.0, 0.01, generator=gen)
    gx = torch.Generator(device=dev).manual_seed(0)
    x = torch.rand(B, 1, 28, 28, device=dev, generator=gx)
    x = (x * (torch.rand(B, 1, 28, 28, device=dev, generator=gx) > 0.8)).requires_grad_(True)
    g = torch.randn(B, 1, 10, device=dev, generator=gx)
    print("[config2] stack forward + backward", flush=True)
    y1 = l1(x)
    y1.retain_grad()
    y2 = l2(y1.reshape(B, 1, 48, 48))
    y2.retain_grad()
    out = head(y2.reshape(B, 1, 800))
    out.backward(g)
    torch.cuda.synchronize()

    def np_(t):
        return t.detach().cpu().numpy().reshape(-1)

    def sparse_check(layer, xin, y, upstream, xgrad, I, O, Nc):
        T = layer.n_detectors()
        E = 1 << Nc
        offs, tg = layer._lut_dm.lookup_connectivity()
        an = layer._detector_anchors.cpu().numpy()
        W = np_(layer._weights)
        idx, md, mi = oracle.check_detectors(xin, an, B, I, T, Nc)
        assert np.array_equal(np_(y), oracle.fill_outputs_sparse(W, idx, offs, tg, B, O, T, E))
        maxg = layer._lut_dm.get_max_forward_groups_per_neuron()
        rxg = oracle.propagate_sparse(W, upstream, idx, md, mi, an, offs, tg, B, I, O, T, Nc, E, 32, maxg)
        rwg = np.zeros(W.size, np.float32)
        oracle.gather_wgrad_sparse(upstream, idx, offs, tg, rwg, B, O, T, E)
        assert np.array_equal(np_(layer._weights.grad), rwg)
        _xg_close(np_(xgrad), rxg, B, I, abs_eps=T * 1e-17)

    # head: dense 800 -> 10, 128 tables of 6 pairs
    Th, Nch, Eh = 128, 6, 64
    ah = head._detector_anchors.cpu().numpy()
    Wh = np_(head._weights)
    hidx, hmd, hmi = oracle.check_detectors(np_(y2), ah, B, 800, Th, Nch)
    assert np.array_equal(np_(out), oracle.fill_outputs_fc(Wh, hidx, B, 10, Th, Eh))
    rxg = oracle.propagate_fc(Wh, np_(g), hidx, hmd, hmi, ah, B, 800, 10, Th, Nch, Eh)
    rwg = np.zeros(Wh.size, np.float32)
    oracle.gather_wgrad_fc(np_(g), hidx, rwg, B, 10, Th, Eh)
    assert np.array_equal(np_(head._weights.grad), rwg)
    _xg_close(np_(y2.grad), rxg, B, 800, abs_eps=Th * 1e-17)
    sparse_check(l2, np_(y1), y2, np_(y2.grad), y1.grad, 2304, 800, 6)
    sparse_check(l1, np_(x), y1, np_(y1.grad), x.grad, 784, 2304, 5)


def test_config2_graph_replay(cuda_device):
    """The config-2 step captured in a HIP graph (as bench.py --config 2 times
    it) and replayed four times, with eager work and a synchronisation before
    each replay.  Every replay must give the eager step's results: the output
    and the head's and layer 2's weight gradients bit for bit; layer 1's weight
    gradient and the input gradient within 1e-5 of each row's largest value
    (their upstream gradients come from fp32 atomics, whose order varies from
    run to run, eager or replayed)."""
    from bench import build_projection_stack
    dev = cuda_device
    B = 128
    l1, l2, head = build_projection_stack(dev)
    gen = torch.Generator(device=dev).manual_seed(3)
    with torch.no_grad():
        for layer in (l1, l2, head):
            layer._weights.normal_(0.0, 0.01, generator=gen)
    gx = torch.Generator(device=dev).manual_seed(1)
    x = torch.rand(B, 1, 28, 28, device=dev, generator=gx)
    x = (x * (torch.rand(B, 1, 28, 28, device=dev, generator=gx) > 0.8)).requires_grad_(True)
    g = torch.randn(B, 1, 10, device=dev, generator=gx)
    params = [l1._weights, l2._weights, head._weights]
    res = {}

    def step():
        for p_ in params:
            p_.grad = None
        x.grad = None
        out = head(l2(l1(x).reshape(B, 1, 48, 48)).reshape(B, 1, 800))
        out.backward(g)
        res["out"] = out

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ref_out = res["out"].detach().clone()
    ref_w = [p_.grad.detach().clone() for p_ in params]
    ref_x = x.grad.detach().clone()
    print("[config2 graph] capture", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    gout, gw, gxg = res["out"], [p_.grad for p_ in params], x.grad
    for rep in range(4):
        with torch.no_grad():
            torch.randn(1 << 20, device=dev).mul_(2.0)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"[config2 graph] replay {rep}", flush=True)
        assert torch.equal(gout, ref_out)
        assert torch.equal(gw[1], ref_w[1]) and torch.equal(gw[2], ref_w[2])
        w1, r1 = gw[0].cpu().numpy(), ref_w[0].cpu().numpy()
        assert np.all(np.abs(w1 - r1) <= 1e-5 * np.abs(r1).max())
        _xg_close(gxg.cpu().numpy(), ref_x.cpu().numpy(), B, 784)


@pytest.mark.parametrize("B", [8, 300])
def test_nan_inputs(oracle, cuda_device, B):
    """NaN inputs through the detector check (the LDS-staged kernel at B = 300,
    the plain one at B = 8): a comparison with a NaN gives bit 0, and a NaN
    first anchor stays the minimum (|NaN| < m is always false, proto:1145-1148).
    Indices, margins (NaN where the oracle has NaN) and margin indices must
    match the oracle bit for bit."""
    from spiky_amd import LUTDataManagerF
    dev = cuda_device
    I, T, Nc, O = 96, 64, 5, 32
    g = torch.Generator().manual_seed(17)
    x = torch.randn(B * I, generator=g)
    x[torch.rand(B * I, generator=g) < 0.1] = float("nan")
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, 32, 32)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    W = torch.randn(T * (1 << Nc) * O, generator=g) * 0.01
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    md = torch.empty(B * T, device=dev)
    mi = torch.empty(B * T, dtype=torch.int32, device=dev)
    dm.forward_step(W.to(dev), B, x.to(dev), anchors.to(dev), out, idx, 0.0, None, md, mi)
    torch.cuda.synchronize()
    ridx, rmd, rmi = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc)
    assert np.isnan(rmd).any()
    assert np.array_equal(idx.cpu().numpy(), ridx)
    gmd = md.cpu().numpy()
    # NaN payloads may differ between the two subtractions; NaN positions may not
    assert np.array_equal(np.isnan(gmd), np.isnan(rmd))
    assert np.array_equal(gmd[~np.isnan(rmd)], rmd[~np.isnan(rmd)])
    assert np.array_equal(mi.cpu().numpy(), rmi)
    assert np.array_equal(out.cpu().numpy(), oracle.fill_outputs_fc(W.numpy(), ridx, B, O, T, 1 << Nc))


@pytest.mark.parametrize("Nc,train", [(8, True), (12, False)])
def test_check_runs_of_sample_groups(oracle, cuda_device, Nc, train):
    """The detector check's workgroups each walk a run of sample groups (here
    4-sample groups, two a run, 750 groups): a partial last group (B = 2999),
    runs past the last group that do nothing, both anchor-register widths, in
    training (margins and their indices) and in evaluation.  Indices, margins
    and margin indices bit-exact against the oracle."""
    from spiky_amd import LUTDataManagerF
    dev = cuda_device
    B, I, T, O = 2999, 4096, 2048, 32
    E = 1 << Nc
    g = torch.Generator().manual_seed(23)
    x = torch.randn(B * I, generator=g)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten()
    dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, 32, 32)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    W = torch.zeros(T * E * O, device=dev)
    out = torch.zeros(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)
    md = torch.empty(B * T, device=dev) if train else None
    mi = torch.empty(B * T, dtype=torch.int32, device=dev) if train else None
    print(f"[check runs] B={B} I={I} T={T} Nc={Nc} train={train}", flush=True)
    dm.forward_step(W, B, x.to(dev), anchors.to(dev), out, idx, 0.0, None, md, mi)
    torch.cuda.synchronize()
    res = oracle.check_detectors(x.numpy(), anchors.numpy(), B, I, T, Nc, train=train)
    ridx = res[0] if train else res
    assert np.array_equal(idx.cpu().numpy(), ridx)
    if train:
        assert np.array_equal(md.cpu().numpy(), res[1])
        assert np.array_equal(mi.cpu().numpy(), res[2])
