"""LUT layers over this library's LUTDataManagerF/I: the Python surface of the
reference's src/spiky/lut/LUTLayer.py (class names, constructor signatures,
method names, tensor shapes, error texts, GradientPolicy semantics and the
LUTForwardFN autograd contract), built on a design of its own.

A layer's sizes and modes are one validated record, _Topology, that every
constructor fills and LUTLayerBasic reads; its legacy attributes (_n_inputs,
_n_detectors, ...) are views of it.  Conv2DLUTLayer and ProjectionLUTLayer
plan their geometry first (_ConvGeometry, _ProjectionGeometry) and then wire
detector and lookup connectivity from the plan.  LUTForwardFN dispatches the
three lookup modes -- single step, sequence concatenation, pair product --
through one table of (forward, backward) routines.

Behaviour that differs from the reference, on purpose:
  * kernels run on torch's current HIP stream and nothing blocks the host
    (the reference synchronises three side streams after every call,
    LUTLayer.py:539-549);
  * the Dense weight gradient is written, not accumulated, so it needs no
    zeros_like pass (LUTLayer.py:864) -- same values;
  * the detector anchors are a registered buffer (they travel with state_dict);
  * in product mode lut_shape() counts the 2^n_anchors rows each table has
    (the reference's Conv2DLUTLayer counts 4^n_anchors there, LUTLayer.py:1299).
"""
from dataclasses import dataclass
from enum import Enum
from typing import List, NamedTuple, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from .lut_data_manager import LUTDataManagerF, LUTDataManagerI
from ..util.chunk_of_connections import ChunkOfConnections, repeat_connections_incrementing_source
from ..util.torch_utils import DenseToSparseConverter
from ..util.synapse_growth import (Conv2DSynapseGrowthHelper, GivenRectanglesSynapseGrowthHelper,
                                   PointSamplingPolicy, PointSamplingType,
                                   RandomRectanglesSynapseGrowthHelper)


class GradientType(Enum):
    """Weight-gradient handling (reference LUTLayer.py:18-22)."""
    Sparse = 0
    Dense = 1
    Internal = 2


@dataclass(frozen=True)
class GradientPolicy:
    type: GradientType
    normalized: bool = False

    def __post_init__(self):
        if self.normalized and self.type == GradientType.Internal:
            raise ValueError("normalized cannot be combined with Internal gradient policy")


@dataclass(frozen=True, order=True)
class SynapseMeta:
    learning_rate: float = 1.0
    min_weight: float = 0.0
    max_weight: float = 1.0
    initial_noise_level: float = 0.0
    initial_weight: float = 0.0

    def __post_init__(self):
        assert 0.0 <= self.learning_rate <= 1.0
        assert self.min_weight <= self.initial_weight <= self.max_weight


# ---------------------------------------------------------------------- shared context
class _BufferPool:
    """Grow-only device tensors keyed by (kind, multi_id): a request returns the
    first `numel` entries of a tensor at least that long, allocated anew only
    when the held one is too short or lives elsewhere."""

    def __init__(self):
        self._held = {}

    def get(self, kind, multi_id, numel, dtype, device, zeroed):
        cur = self._held.get((kind, multi_id))
        if cur is None or cur.numel() < numel or cur.device != device:
            make = torch.zeros if zeroed else torch.empty
            cur = make([numel], dtype=dtype, device=device)
            self._held[(kind, multi_id)] = cur
        return cur[:numel]

    def listing(self, kind):
        ids = sorted(m for k, m in self._held if k == kind)
        out = [None] * (ids[-1] + 1 if ids else 0)
        for m in ids:
            out[m] = self._held[(kind, m)]
        return out

    def move(self, device):
        self._held = {key: t.to(device) for key, t in self._held.items()}


class LUTSharedContext(object):
    """State a model's LUT layers share (reference LUTLayer.py:49-194): the
    Sparse policy's dense gradient buffers and converters, the comparison
    epsilon and the device.  Streams are torch's current stream:
    get_cuda_streams returns the three-handle tensor the data-manager API
    accepts."""

    def __init__(self, do_asserts=False, _cmp_eps=0.0):
        self._pool = _BufferPool()
        self._converters = {}
        self._device = None
        self._do_asserts = do_asserts
        self._cmp_eps = _cmp_eps

    @property
    def _weight_gradients_buffers(self):
        return self._pool.listing("w_grad")

    def _require_device(self, device):
        if self._device is None:
            raise RuntimeError('LUTSharedContext device is None, call to_device(...) first')
        if device is not None and self._device != device:
            raise RuntimeError(f'LUTSharedContext is on {self._device}, but trying to get buffer on {device}')

    def get_weight_gradients_buffer(self, numel, device, multi_id=0):
        """A zeroed fp32 buffer of numel entries; the Sparse policy's converter
        erases what it reads, so the buffer stays zero between steps."""
        self._require_device(device)
        buf = self._pool.get("w_grad", multi_id, numel, torch.float32, self._device, zeroed=True)
        if self._do_asserts:
            assert torch.count_nonzero(buf) == 0
        return buf

    def get_dense_to_sparse_converter(self, multi_id=0):
        """Converter of the Sparse policy's gradients (reference LUTLayer.py:87-94)."""
        return self._converters.setdefault(multi_id, DenseToSparseConverter())

    def get_densify_buffers(self, numel, device, multi_id=0):
        """(indices int64, values fp32) buffers of at least numel entries
        (reference LUTLayer.py:96-99)."""
        self._require_device(None)
        return (self._pool.get("densify_idx", multi_id, numel, torch.int64, device, zeroed=False),
                self._pool.get("densify_val", multi_id, numel, torch.float32, device, zeroed=False))

    def get_cuda_streams(self, device, multi_id=0):
        if device.type != 'cuda':
            return None
        h = torch.cuda.current_stream(device).cuda_stream
        return torch.tensor([h, h, h], dtype=torch.int64)

    def get_cuda_stream(self, device, multi_id=0, stream_index=0):
        if device.type != 'cuda':
            return None
        assert 0 <= stream_index < 3, "stream_index must be between 0 and 2"
        return torch.cuda.current_stream(device)

    def to_device(self, device):
        self._device = _resolve_device(device)
        self._pool.move(self._device)
        return self


def _resolve_device(device):
    dev = device if isinstance(device, torch.device) else torch.device(device)
    if dev.type == 'cuda' and dev.index is None:
        dev = torch.device(f'cuda:{torch.cuda.current_device()}')
    return dev


def _device_index(dev):
    if dev.type == 'cuda':
        return dev.index if dev.index is not None else torch.cuda.current_device()
    return -1


# ---------------------------------------------------------------------- topology
@dataclass(frozen=True)
class _Topology:
    """Sizes and lookup modes of one LUT layer, validated once.  In product
    mode (concatenation_product False) the data manager sees one virtual row
    per pair -- [x_i | x_j | pe], or interleaved when sliced -- and a sequence
    length of 1 (reference LUTLayer.py:306-324)."""
    n_inputs: int
    n_outputs: int
    n_detectors: int
    n_anchors: int
    sequence_length: int
    positional_dim: Optional[int]
    concatenation_product: bool
    sliced: bool
    unified_pe: bool
    fully_connected: bool

    def check(self, n_metas, summation_dtype, policy):
        assert n_metas > 0
        assert self.sequence_length > 0
        rules = (
            (self.sequence_length == 1 and not self.concatenation_product,
             "concatenation_product == False doesn't make sense with sequence_length == 1"),
            (self.sliced and self.concatenation_product,
             "sliced_product_mode == True doesn't make sense in concatenation product mode"),
            (self.sliced and self.n_inputs != self.positional_dim,
             "if sliced_product_mode == True then n_inputs and positional_dim should be equal"),
            (summation_dtype == torch.int32 and policy.type == GradientType.Internal,
             "summation dtype torch.int32 can't be combined with GradientType.Internal"),
        )
        for broken, text in rules:
            if broken:
                raise ValueError(text)
        if self.sequence_length > 1:
            assert self.positional_dim is not None, "positional_dim must be provided when sequence_length > 1"
        else:
            assert self.positional_dim is None, "positional_dim must be None when sequence_length == 1"
        if self.fully_connected:
            assert n_metas == 1, "fully connected mode is not compatible with multiple synapse metas"

    @property
    def pd(self):
        return self.positional_dim or 0

    @property
    def n_virtual(self):
        """Inputs the detectors index: the layer's own, or the product row."""
        return self.n_inputs if self.concatenation_product else 2 * self.n_inputs + self.pd

    @property
    def lut_channels(self):
        return LUTLayerBasic.n_lut_channels(self.n_anchors, self.sequence_length, self.concatenation_product)

    def manager(self, summation_dtype, int_rescaler, capacity, fgs, bgs):
        seq = self.sequence_length if self.concatenation_product else 1
        sizes = (self.n_virtual, self.n_outputs, self.n_detectors, self.n_anchors, seq, self.pd,
                 capacity, fgs, bgs)
        if summation_dtype == torch.float32:
            return LUTDataManagerF(*sizes)
        return LUTDataManagerI(*sizes, int_rescaler)

    def positional_embeddings(self, device, seed):
        """U[-1, 1) positional slices [(S-1) * (1 or T) * pd] from `seed`, or None."""
        if self.sequence_length == 1 or self.pd == 0:
            return None
        gen = None
        if seed is not None:
            gen = torch.Generator(device=device)
            gen.manual_seed(seed)
        per_distance = 1 if self.unified_pe else self.n_detectors
        pe = torch.empty((self.sequence_length - 1) * per_distance * self.pd, dtype=torch.float32,
                         device=device)
        return nn.Parameter(pe.uniform_(-1.0, 1.0, generator=gen))


def _topology_view(field):
    return property(lambda self: getattr(self._topology, field))


class LUTLayerBasic(nn.Module):
    @staticmethod
    def n_lut_channels(n_anchors_per_detector, sequence_length, concatentation_product=True):
        if concatentation_product and sequence_length > 1:
            return 1 << (2 * n_anchors_per_detector)
        return 1 << n_anchors_per_detector

    # the reference's attribute names, read from the topology
    _n_inputs = _topology_view("n_inputs")
    _n_outputs = _topology_view("n_outputs")
    _n_detectors = _topology_view("n_detectors")
    _n_anchors_per_detector = _topology_view("n_anchors")
    _sequence_length = _topology_view("sequence_length")
    _positional_dim = _topology_view("positional_dim")
    _concatenation_product = _topology_view("concatenation_product")
    _sliced_product_mode = _topology_view("sliced")
    _unified_positional_embeddings = _topology_view("unified_pe")
    _is_fully_connected = _topology_view("fully_connected")

    def __init__(self, n_inputs, n_outputs, n_detectors, n_anchors_per_detector, is_fully_connected,
                 sequence_length, synapse_metas: List[SynapseMeta], concatenation_product=True,
                 sliced_product_mode=False, positional_dim=None, unified_pe=False,
                 weights_gradient_policy: GradientPolicy = None,
                 shared_context: LUTSharedContext = None, summation_dtype=torch.float32,
                 _int_rescaler=0.001, _initial_synapse_capacity=None,
                 _forward_group_size: int = 32, _backward_group_size: int = 32, random_seed=None):
        super().__init__()
        topo = _Topology(n_inputs, n_outputs, n_detectors, n_anchors_per_detector, sequence_length,
                         positional_dim, concatenation_product, sliced_product_mode, unified_pe,
                         is_fully_connected)
        policy = weights_gradient_policy or GradientPolicy(GradientType.Dense, normalized=False)
        topo.check(len(synapse_metas), summation_dtype, policy)
        self._topology = topo
        self.device = torch.device("cpu")
        self._multi_id = 0
        self._forward_group_size = _forward_group_size
        self._backward_group_size = _backward_group_size
        self._weights_gradient_policy = policy
        self._external_lr_hook = None
        self._own_shared_context = shared_context is None
        self._shared_context = shared_context if shared_context is not None else \
            LUTSharedContext().to_device(self.device)
        self._positional_embeddings = topo.positional_embeddings(self.device, random_seed)
        capacity = _initial_synapse_capacity
        if capacity is None:
            capacity = topo.lut_channels * n_detectors * n_outputs
        self._lut_dm = topo.manager(summation_dtype, _int_rescaler, capacity, _forward_group_size,
                                    _backward_group_size)
        self._synapse_metas = synapse_metas
        for i, sm in enumerate(synapse_metas):
            m_id = self._lut_dm.register_synapse_meta(
                learning_rate=sm.learning_rate, min_synaptic_weight=sm.min_weight,
                max_synaptic_weight=sm.max_weight, initial_noise_level=sm.initial_noise_level,
                initial_weight=sm.initial_weight)
            assert m_id == i
        self._lut_dm.initialize_neurons(is_fully_connected)
        self._n_lookup_neurons = self._lut_dm.get_number_of_lookup_neurons()
        # neuron ids (reference LUTLayer.py:342-357): inputs (the virtual row in
        # product mode) first, then the detectors; lookup neurons (one per table
        # row) first, then the outputs.  They follow the layer across devices.
        n_virtual = topo.n_virtual
        self._input_neuron_ids = torch.arange(n_virtual, dtype=torch.int32)
        self._detector_neuron_ids = torch.arange(n_virtual, n_virtual + n_detectors, dtype=torch.int32)
        self._lookup_neuron_ids = torch.arange(self._n_lookup_neurons, dtype=torch.int32)
        self._output_neuron_ids = torch.arange(self._n_lookup_neurons, self._n_lookup_neurons + n_outputs,
                                               dtype=torch.int32)
        self._weights = None
        self._lookup_indices_callback = None
        self.register_buffer("_detector_anchors", None)

    # ---------------------------------------------------------------- neuron ids
    def get_input_neuron_ids(self):
        return self._input_neuron_ids

    def get_detector_neuron_ids(self):
        return self._detector_neuron_ids

    def get_lookup_neuron_ids(self):
        return self._lookup_neuron_ids

    def get_output_neuron_ids(self):
        return self._output_neuron_ids

    # ---------------------------------------------------------------- build time
    def add_detector_connections(self, chunk_of_connections: ChunkOfConnections, ids_shift=0,
                                 random_seed: int = None):
        self._lut_dm.add_detector_connections(chunk_of_connections.get_connections().cpu(),
                                              chunk_of_connections.get_single_group_size(),
                                              ids_shift, random_seed)

    def _set_full_detector_connectivity(self):
        """Every detector reads every input: the FC receptive field, set directly
        (the growth engine would produce exactly these ascending lists)."""
        every = list(range(self._topology.n_virtual))
        self._lut_dm._detector_inputs = [every for _ in range(self._n_detectors)]

    def initialize_detectors(self, compact_mode=True, seed=None):
        """Anchors from torch-drawn pair codes (reference LUTLayer.py:373-407):
        compact mode draws one code in [0, n(n-1)) per (detector, slot);
        otherwise each detector's codes are a random permutation of all n(n-1)
        ordered pairs.  The data manager decodes them (prepare_detectors(_compact))."""
        n = self._lut_dm.finalize_detector_connections()
        n_pairs = n * (n - 1)
        assert n_pairs >= self._n_anchors_per_detector
        gen = torch.Generator(device="cpu").manual_seed(seed) if seed is not None else None
        if compact_mode:
            codes = torch.randint(n_pairs, [self._n_detectors, n], dtype=torch.int32, generator=gen)
        else:
            codes = torch.rand(self._n_detectors, n_pairs, generator=gen).argsort(dim=1, stable=True)
        anchors = torch.zeros(self._n_detectors * self._n_anchors_per_detector * 2, dtype=torch.int32)
        self._lut_dm.initialize_detectors(codes.to(torch.int32).flatten().contiguous(), n, anchors,
                                          compact_mode)
        self._detector_anchors = anchors.to(self.device)

    def n_inputs(self):
        return self._n_inputs

    def n_lookup_neurons(self):
        return self._n_lookup_neurons

    def n_outputs(self):
        return self._n_outputs

    def n_detectors(self):
        return self._n_detectors

    def n_anchors_per_detector(self):
        return self._n_anchors_per_detector

    def sequence_length(self):
        return self._sequence_length

    def n_synapses(self):
        if self._is_fully_connected:
            return self._n_lookup_neurons * self._n_outputs
        return self._lut_dm.get_number_of_synapses()

    def input_shape(self):
        return (self._n_outputs,)

    def output_shape(self):
        return (self._n_outputs,)

    def __repr__(self):
        return (f'{type(self).__name__}(inputs={self.n_inputs()}, detectors={self.n_detectors()}, '
                f'anchors per detector={self.n_anchors_per_detector()}, outputs={self.n_outputs()}, '
                f'synapses={self.n_synapses()}, manager={self._lut_dm})')

    def add_lookup_connections(self, chunk_of_connections: ChunkOfConnections, ids_shift=0,
                               random_seed: int = None):
        if self._is_fully_connected:
            raise RuntimeError("Can't add lookup connections in fully connected mode")
        self._lut_dm.add_lookup_connections(chunk_of_connections.get_connections().cpu(),
                                            chunk_of_connections.get_single_group_size(),
                                            ids_shift, random_seed)

    def set_external_learning_rate_hook(self, hook_fn):
        if self._weights_gradient_policy.type != GradientType.Internal:
            raise ValueError("external_learning_rate_hook can only be used with GradientPolicy.Internal")
        if hook_fn is None:
            raise ValueError("external_learning_rate_hook cannot be None when using GradientPolicy.Internal")
        self._external_lr_hook = hook_fn

    def _reset_shared_context(self, new_context):
        self._shared_context = new_context
        self._own_shared_context = False

    def compile_lut(self, shuffle_synapses_random_seed: int = None, _only_trainable_backwards=True,
                    do_normalise_weights=False):
        """Weights (reference LUTLayer.py:490-513).  Fully connected tables:
        initial_weight + noise * U[0,1), clipped to [min, max], from torch's
        global generator, optionally scaled to unit norm per table row and
        stored output-major.  Sparse layers: the data manager's compile orders
        the synapses and draws their weights."""
        if self._is_fully_connected:
            w = self._initial_dense_weights(do_normalise_weights)
        else:
            assert not do_normalise_weights, \
                "weights normalisation is currently supported in fully connected mode only"
            w = torch.zeros([self._lut_dm.get_weights_dimension()], dtype=torch.float32)
            self._lut_dm.to_device(-1)
            self._lut_dm.compile(_only_trainable_backwards, w, shuffle_synapses_random_seed)
        self._weights = nn.Parameter(w.to(self.device))
        self._lut_dm.to_device(_device_index(self.device))

    @torch.no_grad()
    def _initial_dense_weights(self, normalise):
        sm = self._synapse_metas[0]
        noise = torch.rand([self._lut_dm.get_weights_dimension()], dtype=torch.float32, device=self.device)
        w = torch.clamp(noise * sm.initial_noise_level + sm.initial_weight, sm.min_weight, sm.max_weight)
        if normalise:
            rows = w.view(self._n_lookup_neurons, self._n_outputs)
            w = (rows / torch.linalg.vector_norm(rows, dim=-1, keepdim=True)).T.reshape(-1)
        return w

    def get_smallest_distinguishable_fraction(self) -> float:
        return self._lut_dm.get_smallest_distinguishable_fraction()

    def get_epsilon(self) -> float:
        return self._lut_dm.get_epsilon()

    def get_summation_type(self) -> torch.dtype:
        kinds = {'int32': torch.int32, 'float32': torch.float32}
        t = self._lut_dm.get_summations_data_type()
        if t not in kinds:
            raise RuntimeError('Unsupported summations type: ' + t)
        return kinds[t]

    def get_memory_stats(self) -> str:
        return self._lut_dm.get_memory_stats()

    def get_profiling_stats(self) -> str:
        return self._lut_dm.get_profiling_stats()

    def reset_profiler(self):
        self._lut_dm.reset_profiler()

    def _synchronize(self):
        """Kernels are stream-ordered on torch's current stream; nothing to wait for."""
        return None

    def _gradient_densify_buffer_size(self, batch_size):
        """Densify buffer entries for a batch (reference LUTLayer.py:551-565):
        the reference's bound, here capped at the gradient's own size, which no
        count of non-zero words can exceed."""
        per_neuron = self._n_outputs if self._is_fully_connected else \
            self._lut_dm.get_max_forward_groups_per_neuron() * self._forward_group_size
        pairs = 1 if self._sequence_length == 1 else self._sequence_length * (self._sequence_length - 1) // 2
        bound = self._n_detectors * per_neuron * batch_size * pairs
        return min(bound, ((self._weights.numel() + 3) // 4) * 4)

    def _process_gradients(self, target_w_grad, batch_size):
        """Gradient policy post-processing (reference LUTLayer.py:567-609)."""
        policy = self._weights_gradient_policy
        if policy.type == GradientType.Sparse:
            ctx = self._shared_context
            indices, values = ctx.get_dense_to_sparse_converter(self._multi_id).dense_to_sparse_32(
                target_w_grad, erase_input=True,
                densify_buffers=ctx.get_densify_buffers(self._gradient_densify_buffer_size(batch_size),
                                                        self.device, self._multi_id),
                stream=None, decouple=True)
            if indices is None:
                return None
            if policy.normalized:
                values /= values.abs().max().clip(1e-16)
            # the converter's indices ascend, so the tensor is coalesced
            return torch.sparse_coo_tensor(indices=indices.unsqueeze(0), values=values,
                                           size=self._weights.shape, device=self.device,
                                           check_invariants=False, is_coalesced=True,
                                           requires_grad=False)
        if policy.type == GradientType.Dense and policy.normalized:
            target_w_grad /= target_w_grad.abs().max().clip(1e-16)
        return target_w_grad

    def _set_lookup_indices_callback(self, cb):
        assert self._sequence_length == 1
        self._lookup_indices_callback = cb

    # ---------------------------------------------------------------- hot path
    def forward_step(self, x, output=None):
        if not (len(x.shape) == len(self.input_shape()) + 2 and tuple(x.shape[2:]) == tuple(self.input_shape())):
            raise ValueError(f"Input x has invalid shape {x.shape}; expected "
                             f"{(x.shape[0], 1, *self.input_shape())} input_shape={self.input_shape()}")
        assert self._sequence_length == 1
        assert x.device == self.device
        batch_size = x.shape[0]
        assert x.shape[1] == 1, f"Input sequence_length {x.shape[1]} does not match constructor sequence_length 1"
        x = x.contiguous().view(-1)
        external_output = output is not None
        if not external_output:
            output = torch.zeros([batch_size * self._n_outputs], dtype=torch.float32, device=self.device)
        lookup_indices = torch.empty([batch_size * self._n_detectors], dtype=torch.int32, device=self.device)
        if self.training:
            min_anchor_deltas = torch.empty([batch_size * self._n_detectors], dtype=torch.float32,
                                            device=self.device)
            min_anchor_delta_indices = torch.empty([batch_size * self._n_detectors], dtype=torch.int32,
                                                   device=self.device)
        else:
            min_anchor_deltas = None
            min_anchor_delta_indices = None
        self._lut_dm.forward_step(self._weights, batch_size, x, self._detector_anchors, output,
                                  lookup_indices, self._shared_context._cmp_eps, None,
                                  min_anchor_deltas, min_anchor_delta_indices)
        if not external_output and self.training and self._lookup_indices_callback is not None:
            self._lookup_indices_callback(lookup_indices, min_anchor_deltas, min_anchor_delta_indices)
        if self.training:
            result = () if external_output else (output.view((batch_size, 1) + tuple(self.output_shape())),)
            return result + (lookup_indices.view(batch_size, 1, self._n_detectors),
                             min_anchor_deltas.view(batch_size, 1, self._n_detectors),
                             min_anchor_delta_indices.view(batch_size, 1, self._n_detectors))
        return None if external_output else output.view((batch_size, 1) + tuple(self.output_shape()))

    def _weight_grad_target(self):
        if self._weights_gradient_policy.type == GradientType.Internal:
            return None, False
        if self._weights_gradient_policy.type == GradientType.Sparse:
            numel = ((self._weights.numel() + 3) // 4) * 4
            return self._shared_context.get_weight_gradients_buffer(numel, self.device, self._multi_id), False
        return torch.empty_like(self._weights, requires_grad=False), True

    def _external_lr(self):
        if self._weights_gradient_policy.type == GradientType.Internal:
            if self._external_lr_hook is None:
                raise ValueError("external_learning_rate_hook must be set when using GradientPolicy.Internal")
            return self._external_lr_hook(self._weights)
        return -1.0

    def backward_step(self, x, grad_output, lookup_indices, min_anchor_deltas,
                      min_anchor_delta_indices, x_grad=None):
        assert self._sequence_length == 1
        assert x.device == self.device
        source_x_shape = x.shape
        batch_size = source_x_shape[0]
        assert x.shape[1] == 1
        expected_shape = (batch_size, 1) + tuple(self.input_shape())
        assert tuple(x.shape) == expected_shape, f"Expected input shape {expected_shape}, got {x.shape}"
        x = x.contiguous().view(-1)
        assert lookup_indices.shape == (batch_size, 1, self._n_detectors)
        assert min_anchor_deltas.shape == (batch_size, 1, self._n_detectors)
        assert min_anchor_delta_indices.shape == (batch_size, 1, self._n_detectors)
        lookup_indices = lookup_indices.reshape(-1)
        min_anchor_deltas = min_anchor_deltas.reshape(-1)
        min_anchor_delta_indices = min_anchor_delta_indices.reshape(-1)
        external_output = x_grad is not None
        if not external_output:
            x_grad = torch.zeros_like(x)
        target_w_grad, overwrite = self._weight_grad_target()
        assert grad_output.device == self.device
        assert tuple(grad_output.shape) == (batch_size, 1) + tuple(self.output_shape())
        grad_output = grad_output.contiguous().view(-1)
        external_lr = self._external_lr()
        self._lut_dm.backward_backprop(self._weights, batch_size, grad_output, self._detector_anchors,
                                       lookup_indices, min_anchor_deltas, min_anchor_delta_indices,
                                       x_grad, external_lr, target_w_grad, None,
                                       overwrite_weights_gradients=overwrite)
        if not external_output:
            target_w_grad = self._process_gradients(target_w_grad, batch_size) \
                if target_w_grad is not None else None
        result = () if external_output else (x_grad.view(source_x_shape),)
        return result + (target_w_grad,)

    def forward_step_concat(self, x, pos_embeddings, output=None):
        """Sequence-concat forward (reference LUTLayer.py:677-777)."""
        if not (len(x.shape) == len(self.input_shape()) + 2 and tuple(x.shape[2:]) == tuple(self.input_shape())):
            raise ValueError(f"Input x has invalid shape {x.shape}; expected "
                             f"{(x.shape[0], 'S', *self.input_shape())} input_shape={self.input_shape()}")
        assert self._concatenation_product
        assert x.device == self.device
        batch_size, sequence_length = x.shape[0], x.shape[1]
        assert sequence_length == self._sequence_length, \
            f"Input sequence_length {sequence_length} does not match constructor sequence_length {self._sequence_length}"
        x = x.contiguous().view(-1)
        external_output = output is not None
        if not external_output:
            output = torch.zeros([batch_size * sequence_length * self._n_outputs], dtype=torch.float32,
                                 device=self.device)
        n_items = batch_size * sequence_length * self._n_detectors
        lookup_indices = torch.empty([n_items], dtype=torch.int32, device=self.device)
        min_anchor_deltas = min_anchor_delta_indices = None
        if self.training:
            min_anchor_deltas = torch.empty([n_items], dtype=torch.float32, device=self.device)
            min_anchor_delta_indices = torch.empty([n_items], dtype=torch.int32, device=self.device)
        pli = pmd = pmi = None
        if self._positional_dim > 0:
            n_pe = (sequence_length - 1) * self._n_detectors
            pli = torch.empty([n_pe], dtype=torch.int32, device=self.device)
            if self.training:
                pmd = torch.empty([n_pe], dtype=torch.float32, device=self.device)
                pmi = torch.empty([n_pe], dtype=torch.int32, device=self.device)
            pos_embeddings = pos_embeddings.contiguous()
        self._lut_dm.forward_step_concat(self._weights, batch_size, x, self._detector_anchors, output,
                                         lookup_indices, self._shared_context._cmp_eps, pos_embeddings,
                                         pli, min_anchor_deltas, min_anchor_delta_indices, pmd, pmi)
        result = () if external_output else \
            (output.view((batch_size, sequence_length) + tuple(self.output_shape())),)
        if not self.training:
            return None if external_output else result[0]
        shp = (batch_size, sequence_length, self._n_detectors)
        pshp = (sequence_length - 1, self._n_detectors)
        return result + (lookup_indices.view(shp), min_anchor_deltas.view(shp),
                         min_anchor_delta_indices.view(shp),
                         None if pli is None else pli.view(pshp),
                         None if pmd is None else pmd.view(pshp),
                         None if pmi is None else pmi.view(pshp))

    def backward_step_concat(self, x, grad_output, lookup_indices, min_anchor_deltas,
                             min_anchor_delta_indices, positional_lookup_indices, positional_min_deltas,
                             positional_min_delta_indices, x_grad=None):
        """Sequence-concat backward (reference LUTLayer.py:901-1009)."""
        assert x.device == self.device
        assert self._concatenation_product
        source_x_shape = x.shape
        batch_size, sequence_length = x.shape[0], x.shape[1]
        assert sequence_length == self._sequence_length
        shp = (batch_size, sequence_length, self._n_detectors)
        assert tuple(lookup_indices.shape) == shp and tuple(min_anchor_deltas.shape) == shp
        assert tuple(min_anchor_delta_indices.shape) == shp
        x = x.contiguous().view(-1)
        lookup_indices = lookup_indices.reshape(-1)
        min_anchor_deltas = min_anchor_deltas.reshape(-1)
        min_anchor_delta_indices = min_anchor_delta_indices.reshape(-1)
        if self._positional_dim > 0:
            pshp = (sequence_length - 1, self._n_detectors)
            assert tuple(positional_lookup_indices.shape) == pshp
            positional_lookup_indices = positional_lookup_indices.reshape(-1)
            positional_min_deltas = positional_min_deltas.reshape(-1)
            positional_min_delta_indices = positional_min_delta_indices.reshape(-1)
            positional_grad = torch.zeros([(sequence_length - 1) * self._n_detectors * self._positional_dim],
                                          dtype=torch.float32, device=self.device)
        else:
            assert positional_lookup_indices is None
            positional_grad = None
        external_output = x_grad is not None
        if not external_output:
            x_grad = torch.zeros_like(x)
        target_w_grad, overwrite = self._weight_grad_target()
        assert tuple(grad_output.shape) == (batch_size, sequence_length) + tuple(self.output_shape())
        grad_output = grad_output.contiguous().view(-1)
        external_lr = self._external_lr()
        self._lut_dm.backward_backprop_concat(
            self._weights, batch_size, grad_output, self._detector_anchors, lookup_indices,
            min_anchor_deltas, min_anchor_delta_indices, x_grad, external_lr, positional_lookup_indices,
            positional_min_deltas, positional_min_delta_indices, positional_grad, target_w_grad, None,
            overwrite_weights_gradients=overwrite)
        if not external_output:
            target_w_grad = self._process_gradients(target_w_grad, batch_size) \
                if target_w_grad is not None else None
        if self._positional_dim > 0 and self._weights_gradient_policy.normalized:
            positional_grad /= positional_grad.abs().max().clip(1e-16)
        result = () if external_output else (x_grad.view(source_x_shape),)
        return result + (target_w_grad, positional_grad)

    def forward_step_product(self, x, pos_embeddings, output=None):
        """Product-mode forward (reference LUTLayer.py:779-821): every pair
        i < j of a sequence is one lookup per table over [x_i | x_j | pe]."""
        if not (len(x.shape) == len(self.input_shape()) + 2 and tuple(x.shape[2:]) == tuple(self.input_shape())):
            raise ValueError(f"Input x has invalid shape {x.shape}; expected "
                             f"{(x.shape[0], 'S', *self.input_shape())} input_shape={self.input_shape()}")
        assert not self._concatenation_product
        assert x.device == self.device
        batch_size, sequence_length = x.shape[0], x.shape[1]
        assert sequence_length == self._sequence_length, \
            f"Input sequence_length {sequence_length} does not match constructor sequence_length {self._sequence_length}"
        x = x.contiguous().view(-1)
        external_output = output is not None
        if not external_output:
            output = torch.zeros([batch_size * sequence_length * self._n_outputs], dtype=torch.float32,
                                 device=self.device)
        if pos_embeddings is not None:
            pos_embeddings = pos_embeddings.contiguous()
        self._lut_dm.forward_step_product(
            self._weights, batch_size, self._sequence_length, x, x, self._detector_anchors, output,
            self._n_inputs, self._n_inputs, self._sliced_product_mode, self._shared_context._cmp_eps,
            pos_embeddings)
        return None if external_output else \
            output.view((batch_size, sequence_length) + tuple(self.output_shape()))

    def backward_step_product(self, x, pos_embeddings, grad_output, x_grad=None):
        """Product-mode backward (reference LUTLayer.py:1011-1089): input,
        positional and weight gradients from the same pair lookups."""
        assert x.device == self.device
        assert not self._concatenation_product
        source_x_shape = x.shape
        batch_size, sequence_length = x.shape[0], x.shape[1]
        assert sequence_length == self._sequence_length
        expected_shape = (batch_size, sequence_length) + tuple(self.input_shape())
        assert tuple(x.shape) == expected_shape, f"Expected input shape {expected_shape}, got {x.shape}"
        x = x.contiguous().view(-1)
        external_output = x_grad is not None
        if not external_output:
            x_grad = torch.zeros_like(x)
        if self._weights_gradient_policy.type == GradientType.Internal:
            target_w_grad = None
        elif self._weights_gradient_policy.type == GradientType.Sparse:
            numel = ((self._weights.numel() + 3) // 4) * 4
            target_w_grad = self._shared_context.get_weight_gradients_buffer(numel, self.device,
                                                                             self._multi_id)
        else:
            target_w_grad = torch.zeros_like(self._weights, requires_grad=False)
        positional_grad = None
        if self._positional_dim > 0:
            pos_embeddings = pos_embeddings.contiguous()
            positional_grad = torch.zeros_like(pos_embeddings, requires_grad=False)
        assert grad_output.device == self.device
        assert tuple(grad_output.shape) == (batch_size, sequence_length) + tuple(self.output_shape())
        grad_output = grad_output.contiguous().view(-1)
        external_lr = self._external_lr()
        self._lut_dm.backward_backprop_product(
            self._weights, batch_size, self._sequence_length, x, x, self._detector_anchors, grad_output,
            x_grad, x_grad, external_lr, self._n_inputs, self._n_inputs, self._sliced_product_mode,
            self._shared_context._cmp_eps, target_w_grad, pos_embeddings, positional_grad)
        if not external_output and target_w_grad is not None:
            target_w_grad = self._process_gradients(target_w_grad, batch_size)
        if self._positional_dim > 0 and self._weights_gradient_policy.normalized:
            positional_grad /= positional_grad.abs().max().clip(1e-16)
        result = () if external_output else (x_grad.view(source_x_shape),)
        return result + (target_w_grad, positional_grad)

    def to(self, *args, **kwargs):
        super().to(*args, **kwargs)
        target = kwargs.get("device", args[0] if args else None)
        self.device = _resolve_device(target)
        for name in ("_input_neuron_ids", "_detector_neuron_ids", "_lookup_neuron_ids", "_output_neuron_ids"):
            setattr(self, name, getattr(self, name).to(device=self.device))
        self._lut_dm.to_device(_device_index(self.device))
        if self._own_shared_context:
            self._shared_context.to_device(self.device)
        return self

    # ---------------------------------------------------------------- autograd
    def _step_mode(self):
        if self._sequence_length == 1:
            return "single"
        return "concat" if self._concatenation_product else "product"

    class LUTForwardFN(torch.autograd.Function):
        """Autograd entry (reference LUTLayer.py:1117-1181): apply(x, weights,
        positional embeddings or None, layer).  In training the forward saves,
        per mode, (x, indices, min deltas, min-delta indices) for single steps,
        the same plus the positional three for sequence concatenation, and
        (x, positional embeddings) for pair products; the backward returns
        (x_grad, w_grad, pe_grad or None, None)."""

        @staticmethod
        def forward(ctx, x, weights, pos_embeddings, lut_layer):
            mode = lut_layer._step_mode()
            run = _STEP_MODES[mode]
            if not lut_layer.training:
                return run.evaluate(lut_layer, x, pos_embeddings)
            output, saved = run.train(lut_layer, x, pos_embeddings)
            ctx.lut_layer = lut_layer
            ctx.mode = mode
            ctx.save_for_backward(*saved)
            return output

        @staticmethod
        def backward(ctx, grad_output):
            x_grad, w_grad, pe_grad = _STEP_MODES[ctx.mode].backward(ctx.lut_layer, ctx.saved_tensors,
                                                                     grad_output)
            return x_grad, w_grad, pe_grad, None

    def _prepare_positional_embeddings(self):
        """The [(S-1) * T * pd] positional slices the kernels read: the layer's
        own, or one shared slice per distance expanded over the detectors."""
        pe = self._positional_embeddings
        if not self._unified_positional_embeddings:
            return pe
        per_distance = pe.view(self._sequence_length - 1, 1, self._positional_dim)
        return per_distance.expand(-1, self._n_detectors, -1).reshape(-1).contiguous()

    def forward(self, x):
        pe = None if self._sequence_length == 1 else self._prepare_positional_embeddings()
        return LUTLayerBasic.LUTForwardFN.apply(x, self._weights, pe, self)

    def _count_synapses(self, neuron_ids: torch.Tensor):
        if self._is_fully_connected:
            return self._n_lookup_neurons * self._n_outputs
        return self._lut_dm.count_synapses(neuron_ids)

    def _export_synapses(self, neuron_ids, source_ids, weights, target_ids, synapse_metas=None):
        """Fills (source, weight, target) per synapse of the given lookup
        neurons: every output of their table rows when fully connected, the
        data manager's synapse lists otherwise."""
        if not self._is_fully_connected:
            self._lut_dm.export_synapses(self._weights, neuron_ids, source_ids, weights, target_ids,
                                         synapse_metas)
            return
        rows = neuron_ids.long()
        O = self._n_outputs
        source_ids[:] = rows.repeat_interleave(O).to(source_ids.dtype)
        weights[:] = self._weights.detach().view(-1, O).index_select(0, rows.to(self._weights.device)) \
            .reshape(-1).to(weights.device)
        outputs = torch.arange(self._n_lookup_neurons, self._n_lookup_neurons + O, dtype=target_ids.dtype,
                               device=target_ids.device)
        target_ids[:] = outputs.repeat(rows.numel())
        if synapse_metas is not None:
            synapse_metas[:] = 0.0

    def _export_anchors(self):
        if self._detector_anchors is None:
            raise RuntimeError("Detectors are not initialized, call initialize_detectors() first")
        return self._detector_anchors.view(self._n_detectors, self._n_anchors_per_detector, 2)


class _StepMode(NamedTuple):
    """One lookup mode of LUTForwardFN: eval forward, train forward (output and
    tensors to save) and backward (x_grad, w_grad, pe_grad)."""
    evaluate: object
    train: object
    backward: object


def _single_train(layer, x, pe):
    out, li, md, mi = layer.forward_step(x)
    return out, (x, li, md, mi)


def _single_backward(layer, saved, g):
    x, li, md, mi = saved
    x_grad, w_grad = layer.backward_step(x, g, li, md, mi)
    return x_grad, w_grad, None


def _concat_train(layer, x, pe):
    out, *keys = layer.forward_step_concat(x, pe)
    return out, (x, *keys)


def _concat_backward(layer, saved, g):
    x, *keys = saved
    return layer.backward_step_concat(x, g, *keys)


def _product_train(layer, x, pe):
    return layer.forward_step_product(x, pe), (x, pe)


def _product_backward(layer, saved, g):
    x, pe = saved
    return layer.backward_step_product(x, pe, g)


_STEP_MODES = {
    "single": _StepMode(lambda layer, x, pe: layer.forward_step(x), _single_train, _single_backward),
    "concat": _StepMode(lambda layer, x, pe: layer.forward_step_concat(x, pe), _concat_train, _concat_backward),
    "product": _StepMode(lambda layer, x, pe: layer.forward_step_product(x, pe), _product_train,
                         _product_backward),
}


# ---------------------------------------------------------------------- conv geometry
class _ConvGeometry(NamedTuple):
    """Where a Conv2DLUTLayer's detectors look and its lookups project.

    The detectors tile a virtual input (the input itself, or in product mode
    the pair row [x_i | x_j | pe] side by side, or with sliced products the
    three interleaved) with windows of `field` stepping by `stride`, a
    `detectors_shape` block of detectors per window; their grid is
    `lut_shape`.  With a lookup receptive field the tables' rows project, per
    window of that field over the detector grid, onto an output_kernel_shape
    block of outputs (sparse); without one every row reaches every output."""
    virtual_shape: Tuple[int, int]
    field: Tuple[int, int]
    stride: Tuple[int, int]
    lut_shape: Tuple[int, int]
    lut_channels: int
    detector_helper: object
    lookup_helper: object
    output_shape: Tuple[int, int]
    lut_receptive_field_shape: Tuple[int, int, int]

    @property
    def n_detectors(self):
        return self.lut_shape[0] * self.lut_shape[1]

    @property
    def n_outputs(self):
        return self.output_shape[0] * self.output_shape[1]


def _plan_conv(input_shape, n_anchors, detectors_shape, output_kernel_shape, sequence_length,
               receptive_field_shape, receptive_field_stride_shape, lut_receptive_field_shape,
               lut_receptive_field_stride_shape, concatenation_product, sliced, positional_dim):
    h, w = input_shape
    if concatenation_product:
        virtual, widen = (h, w), 1
    elif sliced:
        virtual, widen = (h, 3 * w), 3
    else:
        virtual, widen = (h, 2 * w + (positional_dim or 0)), None
    if receptive_field_shape is None:
        assert receptive_field_stride_shape is None
        field = stride = virtual
    elif widen is None:
        raise ValueError("a receptive field in product mode needs sliced_product_mode == True")
    else:
        field = (receptive_field_shape[0], receptive_field_shape[1] * widen)
        stride = (receptive_field_stride_shape[0], receptive_field_stride_shape[1] * widen)
    detectors = Conv2DSynapseGrowthHelper(virtual[0], virtual[1], field[0], field[1], stride[0], stride[1],
                                          detectors_shape[0], detectors_shape[1])
    lut_shape = (detectors.out_h, detectors.out_w)
    channels = LUTLayerBasic.n_lut_channels(n_anchors, sequence_length, concatenation_product)
    if lut_receptive_field_shape is None:
        assert lut_receptive_field_stride_shape is None
        return _ConvGeometry(virtual, field, stride, lut_shape, channels, detectors, None,
                             tuple(output_kernel_shape), lut_shape + (channels,))
    lookups = Conv2DSynapseGrowthHelper(lut_shape[0], lut_shape[1], lut_receptive_field_shape[0],
                                        lut_receptive_field_shape[1], lut_receptive_field_stride_shape[0],
                                        lut_receptive_field_stride_shape[1], output_kernel_shape[0],
                                        output_kernel_shape[1], n_input_channels=channels)
    return _ConvGeometry(virtual, field, stride, lut_shape, channels, detectors, lookups,
                         (lookups.out_h, lookups.out_w), tuple(lut_receptive_field_shape) + (channels,))


class Conv2DLUTLayer(LUTLayerBasic):
    """Sliding-window detectors over a 2-D input (reference LUTLayer.py:1245-1437)."""

    def __init__(self, input_shape, n_anchors_per_detector, detectors_shape, output_kernel_shape,
                 sequence_length=1, receptive_field_shape=None, receptive_field_stride_shape=None,
                 lut_receptive_field_shape=None, lut_receptive_field_stride_shape=None,
                 synapse_meta=SynapseMeta(), concatenation_product=True, sliced_product_mode=False,
                 positional_dim=None, unified_pe=False, do_normalise_weights=False,
                 weights_gradient_policy: GradientPolicy = None,
                 shared_context: LUTSharedContext = None, summation_dtype=torch.float32,
                 _explicit_anchors=None, _int_rescaler=0.001, _forward_group_size=32,
                 _backward_group_size=32, _max_groups_in_growth_buffer=2 ** 20, random_seed=None,
                 device=None):
        geo = _plan_conv(input_shape, n_anchors_per_detector, detectors_shape, output_kernel_shape,
                         sequence_length, receptive_field_shape, receptive_field_stride_shape,
                         lut_receptive_field_shape, lut_receptive_field_stride_shape,
                         concatenation_product, sliced_product_mode, positional_dim)
        self._input_shape = tuple(input_shape)
        self._output_shape = geo.output_shape
        self._lut_shape = geo.lut_shape + (geo.lut_channels,)
        self._detectors_shape = tuple(detectors_shape)
        self._lut_receptive_field_shape = geo.lut_receptive_field_shape
        sparse = geo.lookup_helper is not None
        super().__init__(n_inputs=input_shape[0] * input_shape[1], n_outputs=geo.n_outputs,
                         n_detectors=geo.n_detectors, n_anchors_per_detector=n_anchors_per_detector,
                         is_fully_connected=not sparse, sequence_length=sequence_length,
                         synapse_metas=[synapse_meta], concatenation_product=concatenation_product,
                         sliced_product_mode=sliced_product_mode, positional_dim=positional_dim,
                         unified_pe=unified_pe, weights_gradient_policy=weights_gradient_policy,
                         shared_context=shared_context, summation_dtype=summation_dtype,
                         _int_rescaler=_int_rescaler,
                         _initial_synapse_capacity=geo.lookup_helper.n_connections() if sparse else 0,
                         _forward_group_size=_forward_group_size,
                         _backward_group_size=_backward_group_size, random_seed=random_seed)
        if device is not None:
            self.to(device=device)
        self._wire_detectors(geo, _explicit_anchors, random_seed,
                             whole_input=receptive_field_shape is None and detectors_shape[0] == 1)
        if sparse:
            self._wire_lookups(geo, random_seed)
        self.compile_lut(do_normalise_weights=do_normalise_weights)

    def _wire_detectors(self, geo, explicit_anchors, seed, whole_input):
        """Anchors: the caller's, or drawn over each detector's window."""
        if explicit_anchors is not None:
            anchors = explicit_anchors.to(dtype=torch.int32).flatten().contiguous()
            # the kernels read x at every anchor id: an id outside the detectors'
            # inputs would read past the sample's row, so it is refused here once
            # (-1, the reference's UINT32_MAX, marks an unused pair)
            expected = self._n_detectors * self._n_anchors_per_detector * 2
            if anchors.numel() != expected:
                raise ValueError(f"_explicit_anchors has {anchors.numel()} ids, expected "
                                 f"n_detectors * n_anchors_per_detector * 2 = {expected}")
            n_virtual = self._topology.n_virtual
            if anchors.numel() and (int(anchors.min()) < -1 or int(anchors.max()) >= n_virtual):
                raise ValueError(f"_explicit_anchors must lie in [0, {n_virtual}) (or be -1 for an "
                                 f"unused pair); got [{int(anchors.min())}, {int(anchors.max())}]")
            self._detector_anchors = anchors.to(device=self.device)
            return
        if whole_input:
            self._set_full_detector_connectivity()
        else:
            chunk = geo.detector_helper.grow_synapses(
                input_ids=self.get_input_neuron_ids().view(geo.virtual_shape) + 1,
                output_ids=self.get_detector_neuron_ids().view(geo.lut_shape) + 1, seed=seed)
            self.add_detector_connections(chunk_of_connections=chunk, ids_shift=-1, random_seed=seed)
        self.initialize_detectors(seed=seed)

    def _wire_lookups(self, geo, seed):
        """Each table row projects onto its lookup window's block of outputs."""
        chunk = geo.lookup_helper.grow_synapses(
            input_ids=self.get_lookup_neuron_ids().view(geo.lut_shape + (geo.lut_channels,)) + 1,
            output_ids=self.get_output_neuron_ids().view(geo.output_shape) + 1, seed=seed)
        self.add_lookup_connections(chunk_of_connections=chunk, ids_shift=-1, random_seed=seed)

    def input_shape(self):
        return self._input_shape

    def output_shape(self):
        return self._output_shape

    def lut_shape(self):
        return self._lut_shape

    def detectors_shape(self):
        return self._detectors_shape

    def lut_receptive_field_shape(self):
        return self._lut_receptive_field_shape

    def __repr__(self):
        return (f'{type(self).__name__}({self.input_shape()} -> {self.output_shape()}, '
                f'{self.detectors_shape()} detectors per window, {self.n_anchors_per_detector()} anchors '
                f'per detector)')


class LUTLayer(Conv2DLUTLayer):
    """Dense LUT layer, n_inputs -> n_outputs through n_detectors tables
    (reference LUTLayer.py:1440-1508): the one-window Conv2DLUTLayer over a
    1 x n_inputs input with a 1 x n_detectors detector block and a
    1 x n_outputs output block."""

    def __init__(self, n_inputs, n_anchors_per_detector, n_detectors, n_outputs, sequence_length=1,
                 synapse_meta=SynapseMeta(), concatenation_product=True, sliced_product_mode=False,
                 positional_dim=None, unified_pe=False, do_normalise_weights=False,
                 weights_gradient_policy: GradientPolicy = None,
                 shared_context: LUTSharedContext = None, summation_dtype=torch.float32,
                 _explicit_anchors=None, _int_rescaler=0.001, _forward_group_size=32,
                 _backward_group_size=32, _max_groups_in_growth_buffer=2 ** 20, random_seed=None,
                 device=None):
        options = dict(locals())
        for own in ("self", "__class__", "n_inputs", "n_detectors", "n_outputs"):
            options.pop(own, None)
        super().__init__(input_shape=(1, n_inputs), detectors_shape=(1, n_detectors),
                         output_kernel_shape=(1, n_outputs), **options)

    def input_shape(self):
        return self._input_shape[1:]

    def output_shape(self):
        return self._output_shape[1:]

    def detectors_shape(self):
        return self._detectors_shape[1:]

    def lut_shape(self):
        return self._lut_shape[1:]

    def lut_receptive_field_shape(self):
        return self._lut_receptive_field_shape[1:]


# ---------------------------------------------------------------------- projection geometry
class _ProjectionGeometry(NamedTuple):
    """Detector groups of a ProjectionLUTLayer: `groups` centres sampled on
    the input (RandomRectanglesSynapseGrowthHelper with the sampling policy),
    `per_group` detectors each anchored inside a `receptive` rectangle around
    its centre, and every lookup row of a group projecting onto the outputs
    inside a `projection` rectangle around the centre scaled to the output."""
    input_shape: Tuple[int, int]
    output_shape: Tuple[int, int]
    groups: int
    per_group: int
    receptive_helper: object
    projection: Tuple[int, int]

    @property
    def scale(self):
        return (self.output_shape[0] / self.input_shape[0], self.output_shape[1] / self.input_shape[1])


class ProjectionLUTLayer(LUTLayerBasic):
    """Detector groups with rectangular receptive fields on a 2-D input, each
    group projecting onto a rectangle of a 2-D output (reference
    LUTLayer.py:1511-1648)."""

    def __init__(self, input_shape, output_shape, n_anchors_per_detector, n_detector_groups,
                 n_detectors_in_group, receptive_shape, projection_shape, synapse_meta=SynapseMeta(),
                 projection_prob=1.0,
                 detectors_sampling_policy: PointSamplingPolicy = PointSamplingPolicy(PointSamplingType.RandomUniform),
                 input_sparsity_mask=None, output_sparsity_mask=None,
                 weights_gradient_policy: GradientPolicy = None,
                 shared_context: LUTSharedContext = None, summation_dtype=torch.float32,
                 _int_rescaler=0.001, _forward_group_size=32, _backward_group_size=32,
                 _max_groups_in_growth_buffer=2 ** 20, random_seed=None, device=None):
        assert n_detector_groups >= 1 and n_detectors_in_group >= 1
        geo = _ProjectionGeometry(
            tuple(input_shape), tuple(output_shape), n_detector_groups, n_detectors_in_group,
            RandomRectanglesSynapseGrowthHelper(
                input_shape[0], input_shape[1], receptive_shape[0], receptive_shape[1], input_shape[0],
                input_shape[1], n_outputs=n_detector_groups, n_out_channels=n_detectors_in_group,
                input_sparsity_mask=input_sparsity_mask, output_sampling_policy=detectors_sampling_policy),
            tuple(projection_shape))
        self._n_detector_groups = n_detector_groups
        self._n_detectors_in_group = n_detectors_in_group
        self._input_shape = geo.input_shape
        self._output_shape = geo.output_shape
        super().__init__(n_inputs=input_shape[0] * input_shape[1], n_outputs=output_shape[0] * output_shape[1],
                         n_detectors=n_detector_groups * n_detectors_in_group,
                         n_anchors_per_detector=n_anchors_per_detector, is_fully_connected=False,
                         sequence_length=1, synapse_metas=[synapse_meta],
                         weights_gradient_policy=weights_gradient_policy, shared_context=shared_context,
                         summation_dtype=summation_dtype, _int_rescaler=_int_rescaler,
                         _forward_group_size=_forward_group_size,
                         _backward_group_size=_backward_group_size, random_seed=random_seed)
        if device is not None:
            self.to(device=device)
        centres = self._anchor_groups(geo, random_seed)
        self._project_groups(geo, centres, projection_prob, output_sparsity_mask, random_seed)
        self.compile_lut()

    def _anchor_groups(self, geo, seed):
        """Grows each group's receptive rectangle, draws the anchors inside it
        and returns the group centres (one row per detector)."""
        chunk, centres = geo.receptive_helper.grow_synapses(
            input_ids=self.get_input_neuron_ids().view(geo.input_shape) + 1,
            output_ids=self.get_detector_neuron_ids() + 1, seed=seed)
        self.add_detector_connections(chunk_of_connections=chunk, ids_shift=-1, random_seed=seed)
        inputs = self._lut_dm._detector_inputs
        self._detector_input_lists = None if inputs is None else [list(v) for v in inputs]
        self.initialize_detectors(seed=seed)
        return centres

    def _project_groups(self, geo, centres, p, output_mask, seed):
        """Every lookup row of a group gets the group's targets: the outputs in
        the projection rectangle around its centre, scaled to the output grid."""
        scaled = centres.clone() * torch.tensor(geo.scale, dtype=centres.dtype)
        self._group_centers = scaled[::geo.per_group].clone()
        helper = GivenRectanglesSynapseGrowthHelper(self._group_centers, geo.projection[0], geo.projection[1],
                                                    geo.output_shape[0], geo.output_shape[1], p=p,
                                                    output_sparsity_mask=output_mask)
        rows_per_group = geo.per_group * LUTLayerBasic.n_lut_channels(self._n_anchors_per_detector, 1)
        first_rows = self.get_lookup_neuron_ids()[::rows_per_group]
        chunk = helper.grow_synapses(input_ids=first_rows + 1,
                                     output_ids=self.get_output_neuron_ids().reshape(geo.output_shape) + 1,
                                     seed=seed)
        chunk = repeat_connections_incrementing_source(chunk, rows_per_group)
        self.add_lookup_connections(chunk_of_connections=chunk, ids_shift=-1, random_seed=seed)

    def input_shape(self):
        return self._input_shape

    def output_shape(self):
        return self._output_shape

    def detectors_shape(self):
        return (self._n_detector_groups, self._n_detectors_in_group)

    def export_weights(self):
        """(weights, source ids, target ids) of every synapse, ordered by target
        and, within a target, by source."""
        n = self.n_synapses()
        sources = torch.zeros([n], dtype=torch.int32)
        targets = torch.zeros([n], dtype=torch.int32)
        weights = torch.zeros([n], dtype=torch.float32)
        self._export_synapses(self.get_lookup_neuron_ids(), sources, weights, targets)
        key = targets.long() * (int(sources.max()) + 1 if n else 1) + sources.long()
        order = torch.argsort(key, stable=True)
        return weights[order], sources[order], targets[order]

    def __repr__(self):
        return (f'ProjectionLUTLayer({self.input_shape()} -> {self.output_shape()}, '
                f'{self._n_detector_groups} groups of {self._n_detectors_in_group} detectors, '
                f'{self.n_anchors_per_detector()} anchors per detector)')
