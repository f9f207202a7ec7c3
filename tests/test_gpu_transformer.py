"""LUTTransformer (reference src/spiky/lut/LUTTransformer.py) on the GPU
against the CPU oracle chained the same way: embedding -> per block
[attention (sequence-concat LUT) + residual, feed-forward LUT on [B*S,1,E] +
residual] -> unembedding LUT.  The logits must be bit-identical (every LUT
output is, and the residual adds are the same fp32 adds); the gradients of
every table and positional embedding are checked through the oracle's
backward chain, fed the same cross-entropy gradient, within 1e-5 of each
gradient's largest magnitude (the unembedding's weight gradient bit for bit).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _anchors(layer):
    return layer._detector_anchors.detach().cpu().numpy()


def _n_embeddings(model):
    e = model.embedding_dim
    return e if isinstance(e, int) else e[0] * e[1]


def oracle_forward(oracle, model, tokens):
    B, S = tokens.shape
    E, V = _n_embeddings(model), model.vocab_size
    z = model.token_embedder.weight.detach().cpu().numpy()[tokens.cpu().numpy()].astype(np.float32)
    saved = []
    for block in model.layers:
        att = block["attention_lut"]
        T, Nc, Npe = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
        W = att._weights.detach().cpu().numpy()
        pe = att._positional_embeddings.detach().cpu().numpy()
        idx, md, mi = oracle.check_detectors(z.reshape(-1), _anchors(att), B * S, E, T, Nc)
        pidx, pmd, pmi = oracle.check_pe(pe, S, T, Npe)
        a = oracle.fill_outputs_seq(W, idx, pidx, B, E, T, S, Nc, Npe).reshape(B, S, E)
        saved.append(("att", att, z.copy(), (idx, md, mi, pidx, pmd, pmi)))
        z = z + a
        ffn = block["ffn"]
        Tf, Ncf = ffn._n_detectors, ffn._n_anchors_per_detector
        Wf = ffn._weights.detach().cpu().numpy()
        fi, fmd, fmi = oracle.check_detectors(z.reshape(-1), _anchors(ffn), B * S, E, Tf, Ncf)
        f = oracle.fill_outputs_fc(Wf, fi, B * S, E, Tf, 1 << Ncf).reshape(B, S, E)
        saved.append(("ffn", ffn, z.copy(), (fi, fmd, fmi)))
        z = z + f
    un = model.unembedder
    Tu, Ncu = un._n_detectors, un._n_anchors_per_detector
    ui, umd, umi = oracle.check_detectors(z.reshape(-1), _anchors(un), B * S, E, Tu, Ncu)
    logits = oracle.fill_outputs_fc(un._weights.detach().cpu().numpy(), ui, B * S, V, Tu, 1 << Ncu)
    saved.append(("un", un, z.copy(), (ui, umd, umi)))
    return logits.reshape(B, S, V), saved


@pytest.mark.parametrize("embedding_dim", [16, (4, 4)])
def test_transformer_forward_backward(oracle, cuda_device, embedding_dim):
    """With a 2-D embedding_dim (h, w) each attention layer is a Conv2DLUTLayer
    over the [h, w] grid whose receptive field covers it
    (LUTTransformer.py:43-67, 226-252): its anchors come from the grid's
    h * w inputs in row-major order and its lookups reach every output, so
    the same oracle chain over E = h * w features applies."""
    from spiky_amd import LUTTransformer
    from spiky_amd.lut.LUTLayer import Conv2DLUTLayer, LUTLayer
    dev = cuda_device
    B, S, V = 3, 9, 16
    model = LUTTransformer(vocab_size=V, embedding_dim=embedding_dim, context_size=S, positional_dim=2,
                           num_layers=2, num_heads=2, n_detectors=3, n_anchors_per_detector=4,
                           n_anchors_per_detector_attention=3, device=dev, seed=11)
    E = _n_embeddings(model)
    # LUTLayer is the one-window Conv2DLUTLayer: compare the exact classes
    kind = LUTLayer if isinstance(embedding_dim, int) else Conv2DLUTLayer
    assert all(type(b["attention_lut"]) is kind for b in model.layers)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for p in (l._weights for l in model._lut_layers()):
            p.copy_((torch.randn(p.numel(), generator=g) * 0.05).to(dev))
    tokens = torch.randint(0, V, (B, S), generator=g).to(dev)
    logits = model(tokens)
    rlogits, saved = oracle_forward(oracle, model, tokens)
    assert np.array_equal(logits.detach().cpu().numpy(), rlogits)

    targets = torch.randint(0, V, (B, S), generator=g)
    # the cross-entropy gradient w.r.t. the (bit-identical) logits, formed once on
    # the CPU and fed to both chains, so the comparison starts from one gradient
    lg = torch.from_numpy(rlogits).requires_grad_(True)
    torch.nn.functional.cross_entropy(lg.reshape(-1, V), targets.reshape(-1)).backward()
    grad_in = lg.grad.numpy().reshape(-1)
    logits.backward(torch.from_numpy(grad_in.reshape(B, S, V)).to(dev))
    torch.cuda.synchronize()
    for kind, layer, zin, keys in reversed(saved):
        W = layer._weights.detach().cpu().numpy()
        T, Nc = layer._n_detectors, layer._n_anchors_per_detector
        O = layer._n_outputs
        if kind in ("un", "ffn"):
            idx, md, mi = keys
            xg = oracle.propagate_fc(W, grad_in, idx, md, mi, _anchors(layer), B * S, E, O, T, Nc, 1 << Nc)
            wg = np.zeros(W.size, np.float32)
            oracle.gather_wgrad_fc(grad_in, idx, wg, B * S, O, T, 1 << Nc)
            peg = None
        else:
            idx, md, mi, pidx, pmd, pmi = keys
            Npe = layer._positional_dim
            xg, peg = oracle.propagate_seq(W, grad_in, idx, md, mi, pidx, pmd, pmi, _anchors(layer), B, E,
                                           O, T, S, Nc, Npe)
            wg = np.zeros(W.size, np.float32)
            oracle.gather_wgrad_seq(grad_in, idx, pidx, wg, B, O, T, S, Nc, Npe)
        gw = layer._weights.grad.cpu().numpy()
        if kind == "un":
            # the first layer of the backward sees the same upstream gradient on
            # both sides, and the weight gradient is formed in the reference's order
            assert np.array_equal(gw, wg), "unembedding weight gradient"
        scale = max(np.abs(wg).max(), 1e-30)
        assert np.abs(gw - wg).max() <= 1e-5 * scale, f"{kind} weight gradient"
        if peg is not None:
            gp = layer._positional_embeddings.grad.cpu().numpy()
            assert np.abs(gp - peg).max() <= 1e-5 * max(np.abs(peg).max(), 1e-30), "positional gradient"
        # residual: the block input's gradient is the output gradient plus the layer's input gradient
        if kind != "un":
            grad_in = (grad_in + xg).astype(np.float32)
        else:
            grad_in = xg

