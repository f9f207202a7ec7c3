"""LUTTransformer at BASELINE config 5's own size on the GPU (reference
src/spiky/lut/LUTTransformer.py:209-271; kernels restated from
lut_runtime_kernels_logic.proto:1807-1904,3629-3835,4188-4304).

The model is bench.py's: batch 32, S = 256, d_model 256, 4 layers x 4 heads,
16 detectors a head (64 attention tables of 2^16 rows, Nc 6, Npe 4),
feed-forward and unembedding tables of 256 rows (Nc 8) over B*S = 8192
samples.  One forward, cross-entropy on next-token targets and backward run
on the GPU with every LUT layer's input, output and gradients captured by
module hooks; the oracle then checks them at this size:

  * forward, chained as the model runs over sequences 0 and 31 (every op is
    per sequence): each layer's output and the logits bit-identical;
  * attention input gradients of sequences 0 and 31, each layer fed the GPU's
    own upstream gradient: within 1e-5 of each row's largest magnitude (plus
    the sub-EPS terms) of the oracle's terms summed in fp64;
  * positional and weight gradients of four tables per attention layer over
    the whole batch: positional within 1e-5 of the largest magnitude, weight
    within the fp32 summation bound n * 2^-24 * sum|terms| of the oracle (the
    reference GPU path adds them with atomics in any order);
  * every attention table's weight gradient: sum over its rows, per column,
    equals sum over (b, j) of j * g[b, j, :] (position j pairs with j earlier
    positions, each pair adds g[b, j] to one row);
  * feed-forward and unembedding layers over the whole batch: weight
    gradients bit-identical, input gradients within the row bar.

At this size the attention layers take the grouped input-gradient pass
(k_seq_group_lists + k_propagate_seq_grp), the LDS-sliced forward
(k_fill_seq_lds) and the sorted weight gradient (k_wgrad_seq_sort).
"""
import concurrent.futures

import numpy as np
import pytest
import torch

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

SEQS = (0, 31)
TABLES = (0, 21, 42, 63)
POOL = 8


def _np(t):
    return t.detach().cpu().numpy()


def _lut_layers(model):
    for li, block in enumerate(model.layers):
        yield f"att{li}", block["attention_lut"]
        yield f"ffn{li}", block["ffn"]
    yield "un", model.unembedder


@pytest.fixture(scope="module")
def run5(cuda_device):
    import bench
    from spiky_amd import LUTTransformer
    dev = cuda_device
    cfg = bench.TRANSFORMER
    B, S, V = bench.TRANSFORMER_BATCH, cfg["context_size"], cfg["vocab_size"]
    print(f"[config5] building LUTTransformer {cfg} batch {B}", flush=True)
    model = LUTTransformer(**cfg, device=dev, seed=1)
    gen = torch.Generator(device=dev).manual_seed(2)
    with torch.no_grad():
        for layer in model._lut_layers():
            layer._weights.normal_(0.0, 0.01, generator=gen)
    # the embedding takes gradients here so that the first attention layer's
    # input gradient reaches its hook as well
    model.token_embedder.weight.requires_grad_(True)
    gt = torch.Generator(device=dev).manual_seed(0)
    stream = torch.randint(0, V, (B, S + 1), device=dev, generator=gt)
    tokens, targets = stream[:, :S].contiguous(), stream[:, 1:].contiguous()
    cap = {}
    hooks = []
    for name, layer in _lut_layers(model):
        cap[name] = {}

        def fwd(mod, inp, out, c=cap[name]):
            c["x"] = inp[0].detach().clone()
            c["y"] = out.detach().clone()

        def bwd(mod, grad_input, grad_output, c=cap[name]):
            c["gy"] = grad_output[0].detach().clone()
            c["gx"] = grad_input[0].detach().clone()

        hooks.append(layer.register_forward_hook(fwd))
        hooks.append(layer.register_full_backward_hook(bwd))
    print("[config5] forward + cross-entropy + backward", flush=True)
    logits = model(tokens)
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, V), targets.reshape(-1))
    loss.backward()
    torch.cuda.synchronize()
    for h in hooks:
        h.remove()
    for name in cap:
        assert set(cap[name]) == {"x", "y", "gy", "gx"}, name
    print(f"[config5] GPU step done, loss {float(loss.detach()):.6f}", flush=True)
    host = {}

    def host_weights(layer):
        # one host copy of each layer's tables, shared by the tests
        key = id(layer)
        if key not in host:
            host[key] = _np(layer._weights)
        return host[key]

    return dict(model=model, cap=cap, logits=logits.detach(), tokens=tokens, B=B, S=S, V=V,
                E=cfg["embedding_dim"], W=host_weights)


def _oracle_forward_sequence(oracle, run, b):
    """The oracle chain over sequence b; returns each layer's output."""
    model, S, E, V, W = run["model"], run["S"], run["E"], run["V"], run["W"]
    z = _np(model.token_embedder.weight)[_np(run["tokens"][b])].astype(np.float32).reshape(-1)
    outs = {}
    for li, block in enumerate(model.layers):
        att = block["attention_lut"]
        T, Nc, Npe = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
        an = _np(att._detector_anchors)
        idx, _, _ = oracle.check_detectors(z, an, S, E, T, Nc)
        pidx, _, _ = oracle.check_pe(_np(att._positional_embeddings), S, T, Npe)
        a = oracle.fill_outputs_seq(W(att), idx, pidx, 1, E, T, S, Nc, Npe)
        outs[f"att{li}"] = a
        z = z + a
        ffn = block["ffn"]
        fi, _, _ = oracle.check_detectors(z, _np(ffn._detector_anchors), S, E, ffn._n_detectors,
                                          ffn._n_anchors_per_detector)
        f = oracle.fill_outputs_fc(W(ffn), fi, S, E, ffn._n_detectors, 1 << ffn._n_anchors_per_detector)
        outs[f"ffn{li}"] = f
        z = z + f
    un = model.unembedder
    ui, _, _ = oracle.check_detectors(z, _np(un._detector_anchors), S, E, un._n_detectors,
                                      un._n_anchors_per_detector)
    outs["un"] = oracle.fill_outputs_fc(W(un), ui, S, V, un._n_detectors, 1 << un._n_anchors_per_detector)
    return outs


def test_config5_forward_chain(oracle, run5):
    S, E, V = run5["S"], run5["E"], run5["V"]
    logits = _np(run5["logits"])
    # the host copies of the tables are made once, before the worker threads
    for _, layer in _lut_layers(run5["model"]):
        run5["W"](layer)
    with concurrent.futures.ThreadPoolExecutor(len(SEQS)) as ex:
        chains = dict(zip(SEQS, ex.map(lambda b: _oracle_forward_sequence(oracle, run5, b), SEQS)))
    for b, outs in chains.items():
        for name, ref in outs.items():
            n_out = V if name == "un" else E
            got = _np(run5["cap"][name]["y"]).reshape(-1, S, n_out)[b].reshape(-1)
            assert np.array_equal(got, ref), f"sequence {b}: {name} output"
        assert np.array_equal(logits[b].reshape(-1), outs["un"]), f"sequence {b}: logits"
    print(f"[config5] forward chain bit-identical for sequences {SEQS}", flush=True)


def _close_rows(gpu, cpu, rows, n_terms, what):
    gpu = np.asarray(gpu).reshape(rows, -1)
    cpu = np.asarray(cpu).reshape(rows, -1)
    bound = 1e-5 * np.abs(cpu).max(axis=1, keepdims=True) + n_terms * 1e-17
    err = np.abs(gpu - cpu)
    assert np.all(err <= bound), f"{what}: max excess {np.max(err - bound)}"


def test_config5_attention_input_gradients(oracle, run5):
    model, cap, S, E, W = run5["model"], run5["cap"], run5["S"], run5["E"], run5["W"]
    jobs = []
    for li, block in enumerate(model.layers):
        att = block["attention_lut"]
        W(att)
        for b in SEQS:
            jobs.append((li, att, b))

    def one(job):
        li, att, b = job
        T, Nc, Npe = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
        c = cap[f"att{li}"]
        x = _np(c["x"]).reshape(-1, S * E)[b]
        gy = _np(c["gy"]).reshape(-1, S * E)[b]
        an = _np(att._detector_anchors)
        idx, md, mi = oracle.check_detectors(x, an, S, E, T, Nc)
        pidx, pmd, pmi = oracle.check_pe(_np(att._positional_embeddings), S, T, Npe)
        rxg, _ = oracle.propagate_seq(W(att), gy, idx, md, mi, pidx, pmd, pmi, an, 1, E, E, T, S, Nc, Npe,
                                      acc64=True)
        return job, rxg

    with concurrent.futures.ThreadPoolExecutor(POOL) as ex:
        for (li, att, b), rxg in ex.map(one, jobs):
            n_ob = (E + att._forward_group_size - 1) // att._forward_group_size
            got = _np(cap[f"att{li}"]["gx"]).reshape(-1, S * E)[b]
            _close_rows(got, rxg, S, S * att._n_detectors * n_ob, f"layer {li} sequence {b} input gradient")
    print(f"[config5] attention input gradients within the row bar for sequences {SEQS}", flush=True)


def _full_batch_keys(oracle, run, li):
    """The oracle's lookup indices and margins of attention layer li over
    the whole batch, [rows][T] each: (idx, md, mi) over B*S rows and
    (pidx, pmd, pmi) over the S - 1 distances."""
    cache = run.setdefault("keys", {})
    if li not in cache:
        att = run["model"].layers[li]["attention_lut"]
        B, S, E = run["B"], run["S"], run["E"]
        T, Nc, Npe = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
        x = _np(run["cap"][f"att{li}"]["x"]).reshape(-1)
        idx, md, mi = oracle.check_detectors(x, _np(att._detector_anchors), B * S, E, T, Nc)
        pidx, pmd, pmi = oracle.check_pe(_np(att._positional_embeddings), S, T, Npe)
        cache[li] = [a.reshape(-1, T) for a in (idx, md, mi, pidx, pmd, pmi)]
    return cache[li]


def test_config5_attention_positional_and_weight_gradients(oracle, run5):
    model, cap, B, S, E, W = run5["model"], run5["cap"], run5["B"], run5["S"], run5["E"], run5["W"]
    jobs = []
    keys = {}
    for li, block in enumerate(model.layers):
        att = block["attention_lut"]
        keys[li] = _full_batch_keys(oracle, run5, li)
        W(att)
        for t in TABLES:
            jobs.append((li, att, t))

    def one(job):
        li, att, t = job
        T, Nc, Npe = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
        gy = _np(cap[f"att{li}"]["gy"]).reshape(-1)
        idx, md, mi, pidx, pmd, pmi = (np.ascontiguousarray(a[:, t]) for a in keys[li])
        an = np.ascontiguousarray(_np(att._detector_anchors).reshape(T, -1)[t])
        Wt = W(att).reshape(T, -1)[t]
        _, rpeg = oracle.propagate_seq(Wt, gy, idx, md, mi, pidx, pmd, pmi, an, B, E, E, 1, S, Nc, Npe,
                                       acc64=True)
        rwg = np.zeros(Wt.size, np.float32)
        oracle.gather_wgrad_seq(gy, idx, pidx, rwg, B, E, 1, S, Nc, Npe)
        mag = np.zeros(Wt.size, np.float32)
        oracle.gather_wgrad_seq(np.abs(gy), idx, pidx, mag, B, E, 1, S, Nc, Npe)
        return job, rpeg, rwg, mag

    with concurrent.futures.ThreadPoolExecutor(POOL) as ex:
        for (li, att, t), rpeg, rwg, mag in ex.map(one, jobs):
            T, Npe = att._n_detectors, att._positional_dim
            pg = _np(att._positional_embeddings.grad).reshape(S - 1, T, Npe)[:, t, :].reshape(-1)
            assert np.abs(pg - rpeg).max() <= 1e-5 * max(np.abs(rpeg).max(), 1e-30), \
                f"layer {li} table {t} positional gradient"
            wg = _np(att._weights.grad.view(T, -1)[t])
            bound = (B * S) * 2.0 ** -24 * mag + 1e-30
            assert np.all(np.abs(wg - rwg) <= bound), \
                f"layer {li} table {t} weight gradient: max excess {np.max(np.abs(wg - rwg) - bound)}"
            assert np.count_nonzero(rwg) > 0
    print(f"[config5] positional and weight gradients of tables {TABLES} match", flush=True)


def test_config5_attention_weight_gradient_column_sums(oracle, run5):
    """Sum over a table's rows of its weight gradient, per column, against
    sum_(b, j) j * g[b, j, :] in fp64 (terms with |g| <= 1e-17 are dropped, as
    the reference does).  Each element is an fp32 sum of at most n terms, so the
    column sum lies within n * 2^-24 * sum_(b, j) j * |g[b, j, :]| of the exact
    one, n being the most pairs one row of the table receives (counted from the
    oracle's lookup indices)."""
    model, cap, B, S, E = run5["model"], run5["cap"], run5["B"], run5["S"], run5["E"]
    dev = run5["logits"].device
    j = torch.arange(S, dtype=torch.float64, device=dev).view(1, S, 1)
    ii, jj = np.triu_indices(S, 1)
    for li, block in enumerate(model.layers):
        att = block["attention_lut"]
        T, Nc, Npe = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
        idx, _, _, pidx, _, _ = _full_batch_keys(oracle, run5, li)
        gy = cap[f"att{li}"]["gy"].reshape(B, S, E).double()
        gy = torch.where(gy.abs() > 1e-17, gy, torch.zeros_like(gy))
        expect = (j * gy).sum(dim=(0, 1))
        magsum = (j * gy.abs()).sum(dim=(0, 1))
        wg = att._weights.grad.view(T, -1, E)
        rows = wg.shape[1]
        for t in range(T):
            got = wg[t].double().sum(dim=0)
            q = idx[:, t].reshape(B, S).astype(np.int64)
            r = (q[:, jj] << (Nc + Npe)) | (q[:, ii] << Npe) | pidx[jj - ii - 1, t].astype(np.int64)
            nmax = int(np.bincount(r.reshape(-1), minlength=rows).max())
            tol = nmax * 2.0 ** -24 * magsum + 1e-30
            assert torch.all((got - expect).abs() <= tol), \
                f"layer {li} table {t}: column sums off by {float((got - expect).abs().max())} (n {nmax})"
    print("[config5] every attention table's weight-gradient column sums match", flush=True)


def test_config5_feed_forward_and_unembedding(oracle, run5):
    model, cap, B, S, E, V, W = (run5[k] for k in ("model", "cap", "B", "S", "E", "V", "W"))
    n = B * S
    for name, layer in _lut_layers(model):
        if name.startswith("att"):
            continue
        T, Nc, O = layer._n_detectors, layer._n_anchors_per_detector, layer._n_outputs
        c = cap[name]
        x, gy = _np(c["x"]).reshape(-1), _np(c["gy"]).reshape(-1)
        an = _np(layer._detector_anchors)
        idx, md, mi = oracle.check_detectors(x, an, n, E, T, Nc)
        Wn = W(layer)
        rxg = oracle.propagate_fc(Wn, gy, idx, md, mi, an, n, E, O, T, Nc, 1 << Nc)
        rwg = np.zeros(Wn.size, np.float32)
        oracle.gather_wgrad_fc(gy, idx, rwg, n, O, T, 1 << Nc)
        assert np.array_equal(_np(layer._weights.grad), rwg), f"{name} weight gradient"
        n_ob = (O + layer._forward_group_size - 1) // layer._forward_group_size
        _close_rows(_np(c["gx"]), rxg, n, T * n_ob, f"{name} input gradient")
    print("[config5] feed-forward and unembedding gradients match over the whole batch", flush=True)
