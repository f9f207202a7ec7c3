"""CPU-side checks of the drop-in boundary: the C-ABI library loads and exports
every entry point include/spiky_lut.h declares; host-side validation raises the
reference's exception types and messages; the receptive-field builder obeys
the invariants the reference's own structural tests check
(src/spiky/lut/tests/test_lut_forward_simple.py:163-219).  No GPU is touched."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "spiky_lut.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(spiky_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from spiky_amd import _native
    L = _native.lib()
    names = header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the Python binding binds each of them
    assert set(names) <= set(_native.exported_symbols())
    assert b"gfx950" in L.spiky_lut_version()


def test_constructor_validation():
    from spiky_amd import LUTDataManagerF, LUTDataManagerI
    with pytest.raises(ValueError, match="n_inputs == 0"):
        LUTDataManagerF(0, 1, 1, 1, 1, 0, 0, 32, 32)
    with pytest.raises(ValueError, match="forward_group_size > MAX_SYNAPSE_GROUP_SIZE"):
        LUTDataManagerF(4, 1, 1, 1, 1, 0, 0, 4096, 32)
    with pytest.raises(ValueError, match="backward_group_size == 0"):
        LUTDataManagerF(4, 1, 1, 1, 1, 0, 0, 32, 0)
    dm = LUTDataManagerI(4, 2, 3, 2, 1, 0, 0, 32, 32, 0.5)
    assert dm.get_summations_data_type() == "int32"
    assert dm.get_smallest_distinguishable_fraction() == pytest.approx((1.0 / 0xFFFFF) / 0.5)
    assert dm.get_number_of_lookup_neurons() == 3 * 4
    with pytest.raises(ValueError, match="learning_rate > 1"):
        dm.register_synapse_meta(1.5, 0, 1, 0, 0)
    assert dm.register_synapse_meta(1.0, 0, 1, 0, 0) == 0
    assert dm.register_synapse_meta(1.0, 0, 1, 0, 0) == 0  # identical meta is reused
    dm.initialize_neurons(True)
    with pytest.raises(ValueError, match="can't register new synapse metas"):
        dm.register_synapse_meta(0.5, 0, 1, 0, 0)
    assert dm.get_weights_dimension() == 12 * 2
    assert dm.get_max_forward_groups_per_neuron() == 1


def test_backward_without_forward_is_value_error():
    """lut.cu:1047-1049: backward before any forward raises 'no active context'.
    Called through the C ABI directly; the check precedes any device access."""
    from spiky_amd import _native
    L = _native.lib()
    h = ctypes.c_void_p()
    _native.check(L.spiky_lut_create(8, 4, 4, 2, 1, 0, 0, 32, 32, 0, 0.0, ctypes.byref(h)))
    try:
        _native.check(L.spiky_lut_register_synapse_meta(h, 1.0, 0.0, 1.0, 0.0, 0.0, None))
        _native.check(L.spiky_lut_initialize_neurons(h, 1))
        dummy = ctypes.c_void_p(16)
        with pytest.raises(ValueError, match="no active context"):
            _native.check(L.spiky_lut_backward_backprop(h, dummy, 1, dummy, dummy, dummy, dummy, dummy,
                                                        dummy, -1.0, dummy, 0, None))
        with pytest.raises(ValueError, match="batch_size == 0"):
            _native.check(L.spiky_lut_forward_step(h, dummy, 0, dummy, dummy, dummy, dummy, 0.0,
                                                   None, None, None))
    finally:
        L.spiky_lut_destroy(h)


def test_cpu_compute_is_refused():
    """There is no CPU fallback: compute on a CPU-resident layer raises."""
    from spiky_amd import LUTLayer
    layer = LUTLayer(16, 3, 8, 4, random_seed=1)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        layer(torch.rand(2, 1, 16))


def test_tensor_checks():
    from spiky_amd.lut.lut_data_manager import check_tensor
    with pytest.raises(RuntimeError, match="must be flat"):
        check_tensor(torch.zeros(2, 2), "t", True, -1)
    with pytest.raises(RuntimeError, match="must have dtype int32"):
        check_tensor(torch.zeros(2), "t", False, -1)
    with pytest.raises(RuntimeError, match="must be contiguous"):
        check_tensor(torch.zeros(4)[::2], "t", True, -1)


def _fc_manager(int_mode=False, seq=1, pd=0):
    from spiky_amd import LUTDataManagerF, LUTDataManagerI
    B_, I, O, T, Nc = 4, 16, 8, 3, 2
    if int_mode:
        dm = LUTDataManagerI(I, O, T, Nc, seq, pd, 0, 32, 32, 0.001)
    else:
        dm = LUTDataManagerF(I, O, T, Nc, seq, pd, 0, 32, 32)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    return dm, (B_, I, O, T, Nc)


def test_int8_forward_validation():
    """forward_step_i8 checks the int8 tables, the optional min-delta outputs and
    the anchors like every other tensor, before any launch."""
    dm, (B, I, O, T, Nc) = _fc_manager(int_mode=True)
    E = 1 << Nc
    f = lambda n: torch.zeros(n)
    i = lambda n: torch.zeros(n, dtype=torch.int32)
    q8 = torch.zeros(T * E * O, dtype=torch.int8)
    args = dict(r_weights_q8=q8, r_scales=f(T), batch_size=B, r_input=f(B * I),
                r_detector_anchors=i(T * Nc * 2), w_output=f(B * O), w_lookup_indices=i(B * T))
    with pytest.raises(RuntimeError, match="r_weights_q8 must have dtype int8"):
        dm.forward_step_i8(**{**args, "r_weights_q8": torch.zeros(T * E * O, dtype=torch.int32)})
    with pytest.raises(RuntimeError, match="r_weights_q8 must be flat"):
        dm.forward_step_i8(**{**args, "r_weights_q8": q8.view(T, -1)})
    with pytest.raises(ValueError, match="r_weights_q8 has"):
        dm.forward_step_i8(**{**args, "r_weights_q8": q8[:-1]})
    with pytest.raises(ValueError, match="r_detector_anchors has"):
        dm.forward_step_i8(**{**args, "r_detector_anchors": i(T * Nc * 2 - 1)})
    with pytest.raises(RuntimeError, match="w_min_anchor_deltas must have real"):
        dm.forward_step_i8(**args, w_min_anchor_deltas=i(B * T), w_min_anchor_delta_indices=i(B * T))
    with pytest.raises(ValueError, match="w_min_anchor_delta_indices has"):
        dm.forward_step_i8(**args, w_min_anchor_deltas=f(B * T), w_min_anchor_delta_indices=i(B * T - 1))
    # every check passed: only the device requirement is left
    with pytest.raises(RuntimeError, match="HIP devices only"):
        dm.forward_step_i8(**args, w_min_anchor_deltas=f(B * T), w_min_anchor_delta_indices=i(B * T))
    # a manager on a GPU refuses host tensors before it reaches a kernel
    dm.to_device(0)
    with pytest.raises(RuntimeError, match="r_weights_q8 must be on CUDA"):
        dm.forward_step_i8(**args)


def test_backward_and_concat_size_validation():
    dm, (B, I, O, T, Nc) = _fc_manager()
    f = lambda n: torch.zeros(n)
    i = lambda n: torch.zeros(n, dtype=torch.int32)
    W = f(dm.get_weights_dimension())
    with pytest.raises(ValueError, match="r_detector_anchors has"):
        dm.backward_backprop(W, B, f(B * O), i(T * Nc * 2 - 2), i(B * T), f(B * T), i(B * T),
                             f(B * I), -1.0, f(W.numel()))
    S, P = 5, 2
    dms, _ = _fc_manager(seq=S, pd=P)
    Ws = f(dms.get_weights_dimension())
    base = dict(r_weights=Ws, batch_size=B, r_input=f(B * S * I), r_detector_anchors=i(T * Nc * 2),
                w_output=f(B * S * O), w_lookup_indices=i(B * S * T), cmp_eps=0.0,
                r_positional_embeddings=f((S - 1) * T * P), w_positional_lookup_indices=i((S - 1) * T))
    with pytest.raises(ValueError, match="w_min_anchor_deltas has"):
        dms.forward_step_concat(**base, w_min_anchor_deltas=f(B * S * T - 1),
                                w_min_anchor_delta_indices=i(B * S * T))
    with pytest.raises(ValueError, match="w_positional_min_delta_indices has"):
        dms.forward_step_concat(**base, w_min_anchor_deltas=f(B * S * T),
                                w_min_anchor_delta_indices=i(B * S * T),
                                w_positional_min_deltas=f((S - 1) * T),
                                w_positional_min_delta_indices=i((S - 1) * T - 1))
    with pytest.raises(ValueError, match="r_detector_anchors has"):
        dms.backward_backprop_concat(Ws, B, f(B * S * O), i(1), i(B * S * T), f(B * S * T),
                                     i(B * S * T), f(B * S * I), -1.0, i((S - 1) * T), f((S - 1) * T),
                                     i((S - 1) * T), f((S - 1) * T * P), f(Ws.numel()))


def test_stream_handles_are_validated_before_launch():
    dm, (B, I, O, T, Nc) = _fc_manager()
    f = lambda n: torch.zeros(n)
    i = lambda n: torch.zeros(n, dtype=torch.int32)
    W = f(dm.get_weights_dimension())
    dm.to_device(0)
    call = lambda h: dm._launch(h, lambda st: 0)
    with pytest.raises(RuntimeError, match="r_stream_handles must have dtype int64"):
        call(torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="at least 3 elements"):
        call(torch.zeros(2, dtype=torch.int64))
    del W


def test_anchor_decode_matches_oracle(oracle):
    """The library's host decode equals the oracle's on random lists."""
    from spiky_amd import _native
    rng = np.random.default_rng(0)
    T, n, Nc = 50, 30, 6
    ids = np.sort(rng.choice(1000, size=(T, n)), axis=1).astype(np.int32).reshape(-1)
    offs = np.arange(T + 1, dtype=np.int64) * n
    codes = rng.integers(0, 2 ** 31 - 1, size=T * n).astype(np.uint32)
    out = np.zeros(T * Nc * 2, np.int32)
    vp = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    _native.check(_native.lib().spiky_lut_decode_anchors_compact(vp(codes), T, n, Nc, vp(offs),
                                                                 vp(ids), vp(out)))
    ref, err = oracle.decode_anchors_compact(codes.astype(np.int64), T, n, Nc, offs, ids)
    assert err == 0 and np.array_equal(out, ref)


def test_fc_layer_anchors_are_the_reference_compact_draw():
    """LUTLayer(random_seed=s) anchors = compact decode of
    torch.randint(I*(I-1), [N_t, I], generator=manual_seed(s)) over the list
    0..I-1 (reference LUTLayer.py:373-407, proto:101-117)."""
    from spiky_amd import LUTLayer
    I, T, Nc = 20, 6, 3
    layer = LUTLayer(I, Nc, T, 4, random_seed=123)
    g = torch.Generator().manual_seed(123)
    codes = torch.randint(I * (I - 1), [T, I], dtype=torch.int32, generator=g).numpy()
    expect = []
    for t in range(T):
        for k in range(Nc):
            c = int(codes[t, k]) % (I * (I - 1))
            a1, a2 = divmod(c, I - 1)
            if a2 >= a1:
                a2 += 1
            expect += [a1, a2]
    assert layer._detector_anchors.tolist() == expect


def test_explicit_anchors_are_range_checked():
    """Explicit anchors are kept as given when every id is an input of the
    layer (or -1, an unused pair), and refused with ValueError otherwise: the
    kernels would read x past the sample's row."""
    from spiky_amd import LUTLayer
    I, T, Nc = 10, 3, 2
    good = torch.tensor([[0, 9], [1, -1], [5, 4], [8, 2], [3, 7], [6, 0]], dtype=torch.int32)
    layer = LUTLayer(I, Nc, T, 4, _explicit_anchors=good)
    assert layer._detector_anchors.tolist() == good.flatten().tolist()
    for bad in ([[0, 10]], [[-2, 3]]):
        a = good.clone()
        a[1] = torch.tensor(bad[0], dtype=torch.int32)
        with pytest.raises(ValueError, match="_explicit_anchors must lie in"):
            LUTLayer(I, Nc, T, 4, _explicit_anchors=a)
    with pytest.raises(ValueError, match="expected n_detectors"):
        LUTLayer(I, Nc, T, 4, _explicit_anchors=good[:4])
    # product mode: the virtual row [x1 | x2 | pe] has 2 * I + pd inputs
    pl = LUTLayer(I, Nc, T, 4, sequence_length=4, positional_dim=1, concatenation_product=False,
                  _explicit_anchors=torch.full((T * Nc * 2,), 2 * I, dtype=torch.int32))
    assert int(pl._detector_anchors.max()) == 2 * I


def test_neuron_ids_are_kept_and_follow_the_layer():
    """The four id ranges are stored once (reference LUTLayer.py:342-357) and
    returned as the same tensors, not rebuilt per call."""
    from spiky_amd import LUTLayer
    layer = LUTLayer(12, 3, 5, 7, random_seed=1)
    assert layer.get_input_neuron_ids() is layer.get_input_neuron_ids()
    assert layer.get_input_neuron_ids().tolist() == list(range(12))
    assert layer.get_detector_neuron_ids().tolist() == list(range(12, 17))
    n_lookup = 5 * 8
    assert layer.get_lookup_neuron_ids().tolist() == list(range(n_lookup))
    assert layer.get_output_neuron_ids().tolist() == list(range(n_lookup, n_lookup + 7))
    assert all(t.dtype == torch.int32 for t in (layer.get_input_neuron_ids(), layer.get_output_neuron_ids()))


def test_chunk_roundtrip():
    from spiky_amd.util.chunk_of_connections import (build_connections, parse_connections,
                                                     repeat_connections_incrementing_source)
    src = [3, 7]
    offs = [0, 5, 6]
    tg = [10, 11, 12, 13, 14, 99]
    ch = build_connections(src, offs, tg, 2)
    s, t = parse_connections(ch.get_connections(), 2)
    assert list(zip(s.tolist(), t.tolist())) == [(3, 10), (3, 11), (3, 12), (3, 13), (3, 14), (7, 99)]
    rep = repeat_connections_incrementing_source(ch, 3)
    s, t = parse_connections(rep.get_connections(), 2)
    pairs = set(zip(s.tolist(), t.tolist()))
    assert (5, 14) in pairs and (9, 99) in pairs and len(pairs) == 18


def test_projection_builder_invariants():
    """Every anchor lies in its detector's receptive rectangle around the group
    centre; every lookup neuron of a group has the group's targets, which lie
    in the projection rectangle around the scaled centre and in the output mask."""
    from spiky_amd import ProjectionLUTLayer
    H = W = 28
    OH, OW = 20, 20
    rh, rw, ph, pw = 5, 5, 4, 4
    groups, per = 30, 6
    out_mask = torch.ones(OH, OW, dtype=torch.bool)
    out_mask[:, :3] = False
    layer = ProjectionLUTLayer((H, W), (OH, OW), 4, groups, per, (rh, rw), (ph, pw),
                               output_sparsity_mask=out_mask, random_seed=9)
    E = 16
    centers = layer._group_centers * torch.tensor([H / OH, W / OW])  # back to input scale
    anchors = layer._export_anchors()
    for t in range(groups * per):
        cx, cy = centers[t // per].tolist()
        for a in anchors[t].reshape(-1).tolist():
            y, x = divmod(a, W)
            assert abs(x - cx) <= (rw - 1) / 2 + 1e-3 and abs(y - cy) <= (rh - 1) / 2 + 1e-3
    offs, tg = layer._lut_dm.lookup_connectivity()
    for grp in range(groups):
        n0 = grp * per * E
        base = tg[offs[n0]:offs[n0 + 1]]
        assert len(base) > 0 and list(base) == sorted(base)
        for n in range(n0, n0 + per * E):
            assert np.array_equal(tg[offs[n]:offs[n + 1]], base)
        cx, cy = layer._group_centers[grp].tolist()
        for o in base.tolist():
            y, x = divmod(o, OW)
            assert out_mask[y, x]
            assert abs(x - cx) <= pw / 2 + 1e-3 and abs(y - cy) <= ph / 2 + 1e-3
        # and no output inside the rectangle (and the mask) is missing
        inside = [y * OW + x for y in range(OH) for x in range(OW)
                  if out_mask[y, x] and abs(x - cx) <= pw / 2 and abs(y - cy) <= ph / 2]
        assert set(inside) <= set(base.tolist())


def test_densify_validation():
    """Host-side checks of the dense -> sparse converter (reference
    torch_utils.py:59-64): they fire before any device work."""
    from spiky_amd import _native
    L = _native.lib()
    # u32 tile offsets (8-byte padded) + u64 chunk offsets (1024 tiles of
    # 4096 words per chunk) + the total slot
    assert L.spiky_densify32_workspace_bytes(0) == 8
    assert L.spiky_densify32_workspace_bytes(4096) == 8 + 16
    assert L.spiky_densify32_workspace_bytes(4096 * 1025) == 4104 + 24
    with pytest.raises(ValueError, match="divisable by 4"):
        _native.check(L.spiky_count_nonzero32(None, 6, None, 0, None, None))
    with pytest.raises(ValueError, match="divisable by 4"):
        _native.check(L.spiky_dense_to_sparse32(None, 10, None, None, 0, None, 0, None, 0, 0, None))
    from spiky_amd.util.torch_utils import DenseToSparseConverter
    conv = DenseToSparseConverter()
    with pytest.raises(ValueError, match="element_size == 4"):
        conv.dense_to_sparse_32(torch.zeros(8, dtype=torch.float64))
    with pytest.raises(ValueError, match="divisable by 4"):
        conv.dense_to_sparse_32(torch.zeros(6))
    with pytest.raises(ValueError, match="GPU device"):
        conv.dense_to_sparse_32(torch.zeros(8))


def test_product_validation():
    """Product-mode host checks (lut.cu:880-891, 986-997; lut_runtime.cu:
    1075-1077) raise before any device access."""
    from spiky_amd import _native
    L = _native.lib()
    d = ctypes.c_void_p(16)

    def make(seq_len, fc=1):
        h = ctypes.c_void_p()
        _native.check(L.spiky_lut_create(8, 4, 4, 2, seq_len, 0, 0, 32, 32, 0, 0.0, ctypes.byref(h)))
        _native.check(L.spiky_lut_register_synapse_meta(h, 1.0, 0.0, 1.0, 0.0, 0.0, None))
        _native.check(L.spiky_lut_initialize_neurons(h, fc))
        return h

    h = make(4)
    try:
        with pytest.raises(ValueError, match="sequence_length should be equal to 1"):
            _native.check(L.spiky_lut_forward_step_product(h, d, 2, 5, d, d, d, d, 4, 4, 0, 0.0, None,
                                                           None))
    finally:
        L.spiky_lut_destroy(h)
    h = make(1)
    try:
        with pytest.raises(ValueError, match="batch_size == 0"):
            _native.check(L.spiky_lut_forward_step_product(h, d, 0, 5, d, d, d, d, 4, 4, 0, 0.0, None,
                                                           None))
        with pytest.raises(ValueError, match="sequence_length == 0"):
            _native.check(L.spiky_lut_forward_step_product(h, d, 2, 0, d, d, d, d, 4, 4, 0, 0.0, None,
                                                           None))
        with pytest.raises(ValueError, match="no active context"):
            _native.check(L.spiky_lut_backward_backprop_product(h, d, 2, 5, d, d, d, d, d, d, -1.0, 4, 4,
                                                                0, 0.0, d, None, None, None))
    finally:
        L.spiky_lut_destroy(h)
    h = make(1, fc=0)
    try:
        with pytest.raises(ValueError, match="sparse connectivity is not compiled"):
            _native.check(L.spiky_lut_forward_step_product(h, d, 2, 5, d, d, d, d, 4, 4, 0, 0.0, None,
                                                           None))
    finally:
        L.spiky_lut_destroy(h)


def test_product_layer_construction():
    """Product-mode layers build on the host: the manager sees the virtual
    row (2n + pd inputs, or 3n sliced) and a sequence length of 1, and the
    reference's argument checks hold (LUTLayer.py:264-274)."""
    from spiky_amd import LUTLayer
    layer = LUTLayer(16, 4, 8, 32, sequence_length=6, concatenation_product=False, positional_dim=4,
                     random_seed=1)
    assert layer._lut_dm.get_number_of_inputs() == 36
    assert layer._weights.numel() == 8 * 16 * 32
    assert layer.lut_shape() == (8, 16)
    a = layer._detector_anchors
    assert a.min() >= 0 and a.max() < 36
    assert layer._positional_embeddings.numel() == 5 * 8 * 4
    sl = LUTLayer(16, 4, 8, 32, sequence_length=6, concatenation_product=False,
                  sliced_product_mode=True, positional_dim=16, random_seed=1)
    assert sl._lut_dm.get_number_of_inputs() == 48
    with pytest.raises(ValueError, match="doesn't make sense with sequence_length == 1"):
        LUTLayer(16, 4, 8, 32, sequence_length=1, concatenation_product=False)
    with pytest.raises(ValueError, match="n_inputs and positional_dim should be equal"):
        LUTLayer(16, 4, 8, 32, sequence_length=6, concatenation_product=False,
                 sliced_product_mode=True, positional_dim=4)
    with pytest.raises(ValueError, match="doesn't make sense in concatenation product mode"):
        LUTLayer(16, 4, 8, 32, sequence_length=6, sliced_product_mode=True, positional_dim=16)


def test_transformer_2d_embedding_construction():
    """A 2-D embedding_dim builds Conv2DLUTLayer attention layers over the grid
    whose one receptive field covers it (LUTTransformer.py:43-67, 111-115):
    fully connected lookups, anchors among the h * w inputs, E = h * w
    features for the embedding, feed-forward and unembedding layers."""
    from spiky_amd import LUTTransformer
    from spiky_amd.lut.LUTLayer import Conv2DLUTLayer, LUTLayer
    m = LUTTransformer(vocab_size=16, embedding_dim=(4, 2), context_size=5, positional_dim=2, num_layers=2,
                       num_heads=2, n_detectors=3, n_anchors_per_detector=4, n_anchors_per_detector_attention=3,
                       seed=11)
    assert m.token_embedder.weight.shape == (16, 8)
    for block in m.layers:
        att = block["attention_lut"]
        assert type(att) is Conv2DLUTLayer and att._is_fully_connected
        assert att.input_shape() == (4, 2) and att.output_shape() == (4, 2)
        assert att._n_detectors == 6 and att._n_outputs == 8
        assert att._weights.numel() == 6 * (1 << (2 * 3 + 2)) * 8
        a = att._detector_anchors
        assert a.min() >= 0 and a.max() < 8
        assert isinstance(block["ffn"], LUTLayer) and block["ffn"]._n_outputs == 8
    assert m.unembedder._lut_dm.get_number_of_inputs() == 8
