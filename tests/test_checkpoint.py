"""Checkpointing by pickling (reference lut.cu:1409-1473, py::pickle at
lut.cu:1652): a layer on the CPU pickles with its data manager's build-time
state and unpickles into an equivalent layer.  CPU-only; the GPU side (refusal
on a device, identical results after a round trip) is in test_gpu_layers.py."""
import pickle

import numpy as np
import torch

from spiky_amd import LUTLayer, LUTTransformer, ProjectionLUTLayer


def _same_state(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    assert sa.keys() == sb.keys()
    for k in sa:
        assert torch.equal(sa[k], sb[k]), k


def test_fc_layer_roundtrip():
    l1 = LUTLayer(64, 4, 32, 16, random_seed=3)
    l2 = pickle.loads(pickle.dumps(l1))
    _same_state(l1, l2)
    assert torch.equal(l1._detector_anchors, l2._detector_anchors)
    dm1, dm2 = l1._lut_dm, l2._lut_dm
    for f in ("get_number_of_inputs", "get_number_of_outputs", "get_number_of_detectors",
              "get_number_of_lookup_neurons", "get_weights_dimension", "get_max_forward_groups_per_neuron"):
        assert getattr(dm1, f)() == getattr(dm2, f)(), f
    assert dm2._h is not None and dm2._h.value != dm1._h.value


def test_int32_summation_roundtrip():
    l1 = LUTLayer(48, 5, 20, 8, random_seed=4, summation_dtype=torch.int32, _int_rescaler=0.25)
    l2 = pickle.loads(pickle.dumps(l1))
    assert l2._lut_dm.get_summations_data_type() == l1._lut_dm.get_summations_data_type()
    assert l2._lut_dm._int_rescaler == 0.25
    _same_state(l1, l2)


def test_projection_layer_roundtrip():
    p1 = ProjectionLUTLayer((28, 28), (24, 24), 5, 36, 8, (5, 5), (4, 4), random_seed=5)
    p2 = pickle.loads(pickle.dumps(p1))
    _same_state(p1, p2)
    (o1, t1), (o2, t2) = p1._lut_dm.lookup_connectivity(), p2._lut_dm.lookup_connectivity()
    assert np.array_equal(o1, o2) and np.array_equal(t1, t2)
    assert p2._lut_dm.get_number_of_synapses() == p1._lut_dm.get_number_of_synapses()


def test_transformer_roundtrip():
    m1 = LUTTransformer(vocab_size=16, embedding_dim=8, context_size=6, positional_dim=2,
                        num_layers=1, num_heads=1, n_detectors=4, n_anchors_per_detector=3)
    m2 = pickle.loads(pickle.dumps(m1))
    _same_state(m1, m2)
