"""LUT layers: the reference's Python surface (src/spiky/lut/LUTLayer.py),
re-implemented over this library's LUTDataManagerF/I.

Kept: class names, constructor signatures, method names, tensor shapes,
GradientPolicy semantics and the LUTForwardFN autograd contract (forward saves
x, lookup indices, min deltas and min-delta indices; backward returns
(x_grad, w_grad, pe_grad, None)).

Changed, on purpose:
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
from typing import List

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


class LUTSharedContext(object):
    """Per-model shared state (reference LUTLayer.py:49-194): the weight
    gradient buffers of the Sparse policy, the comparison epsilon and the
    device.  Streams are torch's current stream; get_cuda_streams returns the
    three-handle tensor the data-manager API accepts."""

    def __init__(self, do_asserts=False, _cmp_eps=0.0):
        self._weight_gradients_buffers = []
        self._densify_indices_buffers = []
        self._densify_values_buffers = []
        self._dense_to_sparse_converters = []
        self._device = None
        self._do_asserts = do_asserts
        self._cmp_eps = _cmp_eps

    def get_weight_gradients_buffer(self, numel, device, multi_id=0):
        if self._device is None:
            raise RuntimeError('LUTSharedContext device is None, call to_device(...) first')
        if self._device != device:
            raise RuntimeError(f'LUTSharedContext is on {self._device}, but trying to get buffer on {device}')
        while len(self._weight_gradients_buffers) <= multi_id:
            self._weight_gradients_buffers.append(None)
        buf = self._weight_gradients_buffers[multi_id]
        if buf is None or buf.numel() < numel:
            buf = torch.zeros([numel], dtype=torch.float32, device=self._device)
            self._weight_gradients_buffers[multi_id] = buf
        if self._do_asserts:
            assert torch.count_nonzero(buf) == 0
        return buf[:numel]

    def get_dense_to_sparse_converter(self, multi_id=0):
        """Converter of the Sparse policy's gradients (reference LUTLayer.py:87-94)."""
        while len(self._dense_to_sparse_converters) <= multi_id:
            self._dense_to_sparse_converters.append(None)
        if self._dense_to_sparse_converters[multi_id] is None:
            self._dense_to_sparse_converters[multi_id] = DenseToSparseConverter()
        return self._dense_to_sparse_converters[multi_id]

    def get_densify_buffers(self, numel, device, multi_id=0):
        """(indices int64, values fp32) buffers of at least numel entries
        (reference LUTLayer.py:96-99)."""
        if self._device is None:
            raise RuntimeError('LUTSharedContext device is None, call to_device(...) first')
        for bufs, dtype in ((self._densify_indices_buffers, torch.int64),
                            (self._densify_values_buffers, torch.float32)):
            while len(bufs) <= multi_id:
                bufs.append(None)
            if bufs[multi_id] is None or bufs[multi_id].numel() < numel or bufs[multi_id].device != device:
                bufs[multi_id] = torch.empty([numel], dtype=dtype, device=device)
        return self._densify_indices_buffers[multi_id], self._densify_values_buffers[multi_id]

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
        dev = device if isinstance(device, torch.device) else torch.device(device)
        if dev.type == 'cuda' and dev.index is None:
            dev = torch.device(f'cuda:{torch.cuda.current_device()}')
        self._device = dev
        self._weight_gradients_buffers = [None if b is None else b.to(dev)
                                          for b in self._weight_gradients_buffers]
        self._densify_indices_buffers = [None if b is None else b.to(dev) for b in self._densify_indices_buffers]
        self._densify_values_buffers = [None if b is None else b.to(dev) for b in self._densify_values_buffers]
        return self


def _device_index(dev):
    if dev.type == 'cuda':
        return dev.index if dev.index is not None else torch.cuda.current_device()
    return -1


class LUTLayerBasic(nn.Module):
    @staticmethod
    def n_lut_channels(n_anchors_per_detector, sequence_length, concatentation_product=True):
        if concatentation_product:
            return 1 << (n_anchors_per_detector * (2 if (sequence_length > 1) else 1))
        return 1 << n_anchors_per_detector

    def _initialize_positional_embeddings(self, random_seed=None):
        if self._sequence_length > 1:
            assert self._positional_dim is not None, "positional_dim must be provided when sequence_length > 1"
            if self._positional_dim > 0:
                g = None
                if random_seed is not None:
                    g = torch.Generator(device=self.device)
                    g.manual_seed(random_seed)
                n = (self._sequence_length - 1) * (1 if self._unified_positional_embeddings
                                                   else self._n_detectors) * self._positional_dim
                pe = torch.empty(n, dtype=torch.float32, device=self.device)
                pe.uniform_(-1.0, 1.0, generator=g)
                self._positional_embeddings = nn.Parameter(pe)
            else:
                self._positional_embeddings = None
        else:
            assert self._positional_dim is None, "positional_dim must be None when sequence_length == 1"
            self._positional_embeddings = None

    def __init__(self, n_inputs, n_outputs, n_detectors, n_anchors_per_detector, is_fully_connected,
                 sequence_length, synapse_metas: List[SynapseMeta], concatenation_product=True,
                 sliced_product_mode=False, positional_dim=None, unified_pe=False,
                 weights_gradient_policy: GradientPolicy = None,
                 shared_context: LUTSharedContext = None, summation_dtype=torch.float32,
                 _int_rescaler=0.001, _initial_synapse_capacity=None,
                 _forward_group_size: int = 32, _backward_group_size: int = 32, random_seed=None):
        super().__init__()
        assert len(synapse_metas) > 0
        assert sequence_length > 0
        self.device = torch.device("cpu")
        self._n_inputs = n_inputs
        self._n_outputs = n_outputs
        self._n_detectors = n_detectors
        self._n_anchors_per_detector = n_anchors_per_detector
        self._is_fully_connected = is_fully_connected
        self._forward_group_size = _forward_group_size
        self._backward_group_size = _backward_group_size
        self._sequence_length = sequence_length
        self._multi_id = 0
        if self._sequence_length == 1 and not concatenation_product:
            raise ValueError("concatenation_product == False doesn't make sense with sequence_length == 1")
        self._concatenation_product = concatenation_product
        self._sliced_product_mode = sliced_product_mode
        if self._sliced_product_mode and concatenation_product:
            raise ValueError("sliced_product_mode == True doesn't make sense in concatenation product mode")
        if self._sliced_product_mode and n_inputs != positional_dim:
            raise ValueError("if sliced_product_mode == True then n_inputs and positional_dim should be equal")
        self._unified_positional_embeddings = unified_pe
        if shared_context is None:
            self._own_shared_context = True
            shared_context = LUTSharedContext()
            shared_context.to_device(self.device)
        else:
            self._own_shared_context = False
        self._shared_context = shared_context
        if weights_gradient_policy is None:
            weights_gradient_policy = GradientPolicy(GradientType.Dense, normalized=False)
        if summation_dtype == torch.int32 and weights_gradient_policy.type == GradientType.Internal:
            raise ValueError("summation dtype torch.int32 can't be combined with GradientType.Internal")
        self._weights_gradient_policy = weights_gradient_policy
        self._external_lr_hook = None
        self._positional_dim = positional_dim
        self._initialize_positional_embeddings(random_seed=random_seed)
        if self._is_fully_connected:
            assert len(synapse_metas) == 1, "fully connected mode is not compatible with multiple synapse metas"
        if _initial_synapse_capacity is None:
            _initial_synapse_capacity = LUTLayerBasic.n_lut_channels(
                n_anchors_per_detector, sequence_length, concatenation_product) * n_detectors * n_outputs
        # product mode: the manager sees one virtual row [x_i | x_j | pe] per
        # pair and a sequence length of 1 (reference LUTLayer.py:306-324)
        n_virtual = n_inputs if concatenation_product else 2 * n_inputs + (positional_dim or 0)
        args = (n_virtual, n_outputs, n_detectors, n_anchors_per_detector,
                sequence_length if concatenation_product else 1,
                positional_dim if positional_dim is not None else 0, _initial_synapse_capacity,
                _forward_group_size, _backward_group_size)
        if summation_dtype == torch.float32:
            self._lut_dm = LUTDataManagerF(*args)
        else:
            self._lut_dm = LUTDataManagerI(*args, _int_rescaler)
        self._n_lookup_neurons = self._lut_dm.get_number_of_lookup_neurons()
        self._synapse_metas = synapse_metas
        for i, sm in enumerate(synapse_metas):
            m_id = self._lut_dm.register_synapse_meta(
                learning_rate=sm.learning_rate, min_synaptic_weight=sm.min_weight,
                max_synaptic_weight=sm.max_weight, initial_noise_level=sm.initial_noise_level,
                initial_weight=sm.initial_weight)
            assert m_id == i
        self._lut_dm.initialize_neurons(is_fully_connected)
        self._input_neuron_ids = torch.arange(0, n_virtual, dtype=torch.int32)
        self._detector_neuron_ids = torch.arange(n_virtual, n_virtual + self._n_detectors,
                                                 dtype=torch.int32)
        self._lookup_neuron_ids = torch.arange(0, self._n_lookup_neurons, dtype=torch.int32)
        self._output_neuron_ids = torch.arange(self._n_lookup_neurons,
                                               self._n_lookup_neurons + n_outputs, dtype=torch.int32)
        self._weights = None
        self._lookup_indices_callback = None
        self.register_buffer("_detector_anchors", None)

    # ---------------------------------------------------------------- build time
    def add_detector_connections(self, chunk_of_connections: ChunkOfConnections, ids_shift=0,
                                 random_seed: int = None):
        self._lut_dm.add_detector_connections(chunk_of_connections.get_connections().cpu(),
                                              chunk_of_connections.get_single_group_size(),
                                              ids_shift, random_seed)

    def _set_full_detector_connectivity(self):
        """Every detector reads every input: the FC receptive field, set directly
        (the growth engine would produce exactly these ascending lists)."""
        dm = self._lut_dm
        n = self._input_neuron_ids.numel()
        dm._detector_inputs = [list(range(n)) for _ in range(self._n_detectors)]

    def initialize_detectors(self, compact_mode=True, seed=None):
        """Anchors from torch-generated pair codes (reference LUTLayer.py:373-407)."""
        max_n = self._lut_dm.finalize_detector_connections()
        assert max_n * (max_n - 1) >= self._n_anchors_per_detector
        g = None
        if seed is not None:
            g = torch.Generator(device="cpu")
            g.manual_seed(seed)
        anchors = torch.zeros(self._n_detectors * self._n_anchors_per_detector * 2, dtype=torch.int32)
        if compact_mode:
            codes = torch.randint(max_n * (max_n - 1), [self._n_detectors, max_n], dtype=torch.int32,
                                  generator=g)
        else:
            noise = torch.rand(self._n_detectors, max_n * (max_n - 1), generator=g)
            codes = noise.argsort(dim=1, stable=True).to(dtype=torch.int32)
        self._lut_dm.initialize_detectors(codes.flatten().contiguous(), max_n, anchors, compact_mode)
        self._detector_anchors = anchors.to(self.device)

    def get_input_neuron_ids(self):
        return self._input_neuron_ids

    def get_detector_neuron_ids(self):
        return self._detector_neuron_ids

    def get_lookup_neuron_ids(self):
        return self._lookup_neuron_ids

    def get_output_neuron_ids(self):
        return self._output_neuron_ids

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
        return (f'LUTLayerBasic({self.n_inputs()} inputs, {self.n_detectors()} detectors, '
                f'{self.n_anchors_per_detector()} anchors per detector, {self.n_outputs()} outputs, '
                f'{self.n_synapses()} synapses, {self._lut_dm})')

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
        """Weights (reference LUTLayer.py:490-513): FC gets
        U[0,1)*noise + initial_weight clipped to [min, max] from the global torch
        RNG; sparse layers get theirs from the data manager's compile."""
        n_weights = self._lut_dm.get_weights_dimension()
        with torch.no_grad():
            if self._is_fully_connected:
                sm = self._synapse_metas[0]
                w = torch.rand([n_weights], dtype=torch.float32, device=self.device)
                w *= sm.initial_noise_level
                w += sm.initial_weight
                w.clip_(sm.min_weight, sm.max_weight)
                if do_normalise_weights:
                    w = w.view(self._n_lookup_neurons, self._n_outputs)
                    w /= w.norm(dim=-1, keepdim=True)
                    w = w.T.flatten()
            else:
                assert not do_normalise_weights, \
                    "weights normalisation is currently supported in fully connected mode only"
                w = torch.zeros([n_weights], dtype=torch.float32)
                self._lut_dm.to_device(-1)
                self._lut_dm.compile(_only_trainable_backwards, w, shuffle_synapses_random_seed)
        self._weights = nn.Parameter(w.to(self.device))
        self._lut_dm.to_device(_device_index(self.device))

    def get_smallest_distinguishable_fraction(self) -> float:
        return self._lut_dm.get_smallest_distinguishable_fraction()

    def get_epsilon(self) -> float:
        return self._lut_dm.get_epsilon()

    def get_summation_type(self) -> torch.dtype:
        t = self._lut_dm.get_summations_data_type()
        if t == 'int32':
            return torch.int32
        if t == 'float32':
            return torch.float32
        raise RuntimeError('Unsupported summations type: ' + t)

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
        if self._is_fully_connected:
            per_neuron = self._n_outputs
        else:
            per_neuron = self._lut_dm.get_max_forward_groups_per_neuron() * self._forward_group_size
        n = self._n_detectors * per_neuron * batch_size
        if self._sequence_length != 1:
            n *= self._sequence_length * (self._sequence_length - 1) // 2
        return min(n, ((self._weights.numel() + 3) // 4) * 4)

    def _process_gradients(self, target_w_grad, batch_size):
        """Gradient policy post-processing (reference LUTLayer.py:567-609)."""
        if self._weights_gradient_policy.type == GradientType.Sparse:
            converter = self._shared_context.get_dense_to_sparse_converter(self._multi_id)
            indices, values = converter.dense_to_sparse_32(
                target_w_grad, erase_input=True,
                densify_buffers=self._shared_context.get_densify_buffers(
                    self._gradient_densify_buffer_size(batch_size), self.device, self._multi_id),
                stream=None, decouple=True)
            if indices is None:
                return None
            if self._weights_gradient_policy.normalized:
                values /= values.abs().max().clip(1e-16)
            # the converter's indices ascend, so the tensor is coalesced
            return torch.sparse_coo_tensor(indices=indices.unsqueeze(0), values=values,
                                           size=self._weights.shape, device=self.device,
                                           check_invariants=False, is_coalesced=True,
                                           requires_grad=False)
        if self._weights_gradient_policy.type == GradientType.Dense and self._weights_gradient_policy.normalized:
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
        device = kwargs.get("device", None)
        if device is None and len(args) > 0:
            device = args[0]
        dev = torch.device(device)
        if dev.type == 'cuda' and dev.index is None:
            dev = torch.device(f'cuda:{torch.cuda.current_device()}')
        self.device = dev
        self._lut_dm.to_device(_device_index(dev))
        if self._own_shared_context:
            self._shared_context.to_device(self.device)
        return self

    class LUTForwardFN(torch.autograd.Function):
        """Autograd entry (reference LUTLayer.py:1117-1181)."""

        @staticmethod
        def forward(ctx, *args, **kwargs):
            x, _, pos_embeddings, lut_layer = args
            if lut_layer.training:
                ctx.lut_layer = lut_layer
                if lut_layer._sequence_length == 1:
                    output, li, md, mi = lut_layer.forward_step(x)
                    ctx.save_for_backward(x, li, md, mi)
                elif lut_layer._concatenation_product:
                    (output, li, md, mi, pli, pmd, pmi) = lut_layer.forward_step_concat(x, pos_embeddings)
                    ctx.save_for_backward(x, li, md, mi, pli, pmd, pmi)
                else:
                    output = lut_layer.forward_step_product(x, pos_embeddings)
                    ctx.save_for_backward(x, pos_embeddings)
                return output
            if lut_layer._sequence_length == 1:
                return lut_layer.forward_step(x)
            if lut_layer._concatenation_product:
                return lut_layer.forward_step_concat(x, pos_embeddings)
            return lut_layer.forward_step_product(x, pos_embeddings)

        @staticmethod
        def backward(ctx, *grad_outputs):
            (grad_output,) = grad_outputs
            if ctx.lut_layer._sequence_length == 1:
                (x, li, md, mi) = ctx.saved_tensors
                x_grad, w_grad = ctx.lut_layer.backward_step(x, grad_output, li, md, mi)
                return x_grad, w_grad, None, None
            if not ctx.lut_layer._concatenation_product:
                (x, pos_embeddings) = ctx.saved_tensors
                x_grad, w_grad, pe_grad = ctx.lut_layer.backward_step_product(x, pos_embeddings,
                                                                              grad_output)
                return x_grad, w_grad, pe_grad, None
            (x, li, md, mi, pli, pmd, pmi) = ctx.saved_tensors
            x_grad, w_grad, pe_grad = ctx.lut_layer.backward_step_concat(x, grad_output, li, md, mi,
                                                                         pli, pmd, pmi)
            return x_grad, w_grad, pe_grad, None

    def _prepare_positional_embeddings(self):
        if self._unified_positional_embeddings:
            return self._positional_embeddings.reshape(self._sequence_length - 1, 1, self._positional_dim) \
                .repeat(1, self._n_detectors, 1).flatten().contiguous()
        return self._positional_embeddings

    def forward(self, x):
        if self._sequence_length == 1:
            return LUTLayerBasic.LUTForwardFN.apply(x, self._weights, None, self)
        return LUTLayerBasic.LUTForwardFN.apply(x, self._weights, self._prepare_positional_embeddings(), self)

    def _count_synapses(self, neuron_ids: torch.Tensor):
        if self._is_fully_connected:
            return self._n_lookup_neurons * self._n_outputs
        return self._lut_dm.count_synapses(neuron_ids)

    def _export_synapses(self, neuron_ids, source_ids, weights, target_ids, synapse_metas=None):
        if self._is_fully_connected:
            source_ids[:] = neuron_ids.view(neuron_ids.numel(), -1).repeat(1, self._n_outputs).flatten()
            weights[:] = self._weights.view(self._n_lookup_neurons, self._n_outputs)[neuron_ids.long()].flatten()
            target_ids[:] = torch.arange(self._n_outputs, device=target_ids.device,
                                         dtype=torch.int32).repeat(neuron_ids.numel())
            target_ids += self._n_lookup_neurons
            if synapse_metas is not None:
                synapse_metas[:] = 0.0
        else:
            self._lut_dm.export_synapses(self._weights, neuron_ids, source_ids, weights, target_ids,
                                         synapse_metas)

    def _export_anchors(self):
        if self._detector_anchors is None:
            raise RuntimeError("Detectors are not initialized, call initialize_detectors() first")
        return self._detector_anchors.view(self._n_detectors, self._n_anchors_per_detector, 2)


class Conv2DLUTLayer(LUTLayerBasic):
    """Sliding-window detectors (reference LUTLayer.py:1245-1437)."""

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
        # detectors see the virtual row of product mode: [x_i | x_j | pe], or
        # sliced, x_i x_j pe interleaved (reference LUTLayer.py:1273-1292)
        if concatenation_product:
            input_shape_ex = tuple(input_shape)
        elif sliced_product_mode:
            input_shape_ex = (input_shape[0], input_shape[1] * 3)
        else:
            input_shape_ex = (input_shape[0], input_shape[1] * 2 + (positional_dim or 0))
        if receptive_field_shape is None:
            assert receptive_field_stride_shape is None
            rf, rs = input_shape_ex, input_shape_ex
        elif concatenation_product:
            rf, rs = receptive_field_shape, receptive_field_stride_shape
        elif sliced_product_mode:
            rf = (receptive_field_shape[0], receptive_field_shape[1] * 3)
            rs = (receptive_field_stride_shape[0], receptive_field_stride_shape[1] * 3)
        else:
            raise ValueError("a receptive field in product mode needs sliced_product_mode == True")
        c_helper_1 = Conv2DSynapseGrowthHelper(input_shape_ex[0], input_shape_ex[1], rf[0], rf[1],
                                               rs[0], rs[1], detectors_shape[0], detectors_shape[1])
        lut_shape = c_helper_1.out_h, c_helper_1.out_w
        n_lut_channels = LUTLayerBasic.n_lut_channels(n_anchors_per_detector, sequence_length,
                                                      concatenation_product)
        n_inputs = input_shape[0] * input_shape[1]
        n_detectors = lut_shape[0] * lut_shape[1]
        if lut_receptive_field_shape is not None:
            c_helper_2 = Conv2DSynapseGrowthHelper(lut_shape[0], lut_shape[1], lut_receptive_field_shape[0],
                                                   lut_receptive_field_shape[1],
                                                   lut_receptive_field_stride_shape[0],
                                                   lut_receptive_field_stride_shape[1],
                                                   output_kernel_shape[0], output_kernel_shape[1],
                                                   n_input_channels=n_lut_channels)
            n_outputs = c_helper_2.out_h * c_helper_2.out_w
            self._lut_receptive_field_shape = tuple(lut_receptive_field_shape) + (n_lut_channels,)
            self._output_shape = (c_helper_2.out_h, c_helper_2.out_w)
        else:
            assert lut_receptive_field_stride_shape is None
            c_helper_2 = None
            n_outputs = output_kernel_shape[0] * output_kernel_shape[1]
            self._lut_receptive_field_shape = tuple(lut_shape) + (n_lut_channels,)
            self._output_shape = tuple(output_kernel_shape)
        self._input_shape = tuple(input_shape)
        self._lut_shape = tuple(lut_shape) + (n_lut_channels,)
        self._detectors_shape = tuple(detectors_shape)
        super().__init__(n_inputs=n_inputs, n_outputs=n_outputs, n_detectors=n_detectors,
                         n_anchors_per_detector=n_anchors_per_detector,
                         is_fully_connected=c_helper_2 is None, sequence_length=sequence_length,
                         synapse_metas=[synapse_meta], concatenation_product=concatenation_product,
                         sliced_product_mode=sliced_product_mode, positional_dim=positional_dim,
                         unified_pe=unified_pe, weights_gradient_policy=weights_gradient_policy,
                         shared_context=shared_context, summation_dtype=summation_dtype,
                         _int_rescaler=_int_rescaler,
                         _initial_synapse_capacity=0 if c_helper_2 is None else c_helper_2.n_connections(),
                         _forward_group_size=_forward_group_size,
                         _backward_group_size=_backward_group_size, random_seed=random_seed)
        if device is not None:
            self.to(device=device)
        if _explicit_anchors is None:
            whole_input = (receptive_field_shape is None and detectors_shape[0] == 1)
            if whole_input:
                self._set_full_detector_connectivity()
            else:
                connections = c_helper_1.grow_synapses(
                    input_ids=self.get_input_neuron_ids().view(input_shape_ex) + 1,
                    output_ids=self.get_detector_neuron_ids().view(lut_shape[0], lut_shape[1]) + 1,
                    seed=random_seed)
                self.add_detector_connections(chunk_of_connections=connections, ids_shift=-1,
                                              random_seed=random_seed)
            self.initialize_detectors(seed=random_seed)
        else:
            self._detector_anchors = _explicit_anchors.to(device=self.device, dtype=torch.int32) \
                .flatten().contiguous()
        if c_helper_2 is not None:
            connections = c_helper_2.grow_synapses(
                input_ids=self.get_lookup_neuron_ids().view(tuple(lut_shape) + (n_lut_channels,)) + 1,
                output_ids=self.get_output_neuron_ids().view(c_helper_2.out_h, c_helper_2.out_w) + 1,
                seed=random_seed)
            self.add_lookup_connections(chunk_of_connections=connections, ids_shift=-1,
                                        random_seed=random_seed)
        self.compile_lut(do_normalise_weights=do_normalise_weights)

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
        return (f'Conv2DLUTLayer(input_shape={self.input_shape()}, output_shape={self.output_shape()}, '
                f'detectors_shape={self.detectors_shape()}, '
                f'n_anchors_per_detector={self.n_anchors_per_detector()})')


class LUTLayer(Conv2DLUTLayer):
    """Dense LUT layer: n_inputs -> n_outputs through n_detectors tables
    (reference LUTLayer.py:1440-1508)."""

    def __init__(self, n_inputs, n_anchors_per_detector, n_detectors, n_outputs, sequence_length=1,
                 synapse_meta=SynapseMeta(), concatenation_product=True, sliced_product_mode=False,
                 positional_dim=None, unified_pe=False, do_normalise_weights=False,
                 weights_gradient_policy: GradientPolicy = None,
                 shared_context: LUTSharedContext = None, summation_dtype=torch.float32,
                 _explicit_anchors=None, _int_rescaler=0.001, _forward_group_size=32,
                 _backward_group_size=32, _max_groups_in_growth_buffer=2 ** 20, random_seed=None,
                 device=None):
        super().__init__(input_shape=(1, n_inputs), n_anchors_per_detector=n_anchors_per_detector,
                         detectors_shape=(1, n_detectors), output_kernel_shape=(1, n_outputs),
                         sequence_length=sequence_length, synapse_meta=synapse_meta,
                         concatenation_product=concatenation_product,
                         sliced_product_mode=sliced_product_mode, positional_dim=positional_dim,
                         unified_pe=unified_pe, do_normalise_weights=do_normalise_weights,
                         weights_gradient_policy=weights_gradient_policy,
                         shared_context=shared_context, summation_dtype=summation_dtype,
                         _explicit_anchors=_explicit_anchors, _int_rescaler=_int_rescaler,
                         _forward_group_size=_forward_group_size,
                         _backward_group_size=_backward_group_size,
                         _max_groups_in_growth_buffer=_max_groups_in_growth_buffer,
                         random_seed=random_seed, device=device)

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

    def __repr__(self):
        return (f'LUTLayer({self.n_inputs()} inputs, {self.n_detectors()} detectors, '
                f'{self.n_outputs()} outputs, {self.n_anchors_per_detector()} anchors per detector)')


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
        assert n_detector_groups >= 1
        assert n_detectors_in_group >= 1
        self._n_detector_groups = n_detector_groups
        self._n_detectors_in_group = n_detectors_in_group
        c_helper = RandomRectanglesSynapseGrowthHelper(
            input_shape[0], input_shape[1], receptive_shape[0], receptive_shape[1], input_shape[0],
            input_shape[1], n_outputs=n_detector_groups, n_out_channels=n_detectors_in_group,
            input_sparsity_mask=input_sparsity_mask, output_sampling_policy=detectors_sampling_policy)
        n_inputs = input_shape[0] * input_shape[1]
        n_outputs = output_shape[0] * output_shape[1]
        self._input_shape = tuple(input_shape)
        self._output_shape = tuple(output_shape)
        n_lut_channels = LUTLayerBasic.n_lut_channels(n_anchors_per_detector, 1)
        super().__init__(n_inputs=n_inputs, n_outputs=n_outputs,
                         n_detectors=n_detector_groups * n_detectors_in_group,
                         n_anchors_per_detector=n_anchors_per_detector, is_fully_connected=False,
                         sequence_length=1, synapse_metas=[synapse_meta],
                         weights_gradient_policy=weights_gradient_policy, shared_context=shared_context,
                         summation_dtype=summation_dtype, _int_rescaler=_int_rescaler,
                         _forward_group_size=_forward_group_size,
                         _backward_group_size=_backward_group_size, random_seed=random_seed)
        if device is not None:
            self.to(device=device)
        connections, group_centers = c_helper.grow_synapses(
            input_ids=self.get_input_neuron_ids().view(input_shape) + 1,
            output_ids=self.get_detector_neuron_ids() + 1, seed=random_seed)
        self.add_detector_connections(chunk_of_connections=connections, ids_shift=-1,
                                      random_seed=random_seed)
        self._detector_input_lists = [list(v) for v in self._lut_dm._detector_inputs] \
            if self._lut_dm._detector_inputs is not None else None
        self.initialize_detectors(seed=random_seed)
        group_centers = group_centers.clone()
        group_centers[:, 0] *= output_shape[0] / input_shape[0]
        group_centers[:, 1] *= output_shape[1] / input_shape[1]
        self._group_centers = group_centers[::n_detectors_in_group].clone()
        c_helper = GivenRectanglesSynapseGrowthHelper(self._group_centers, projection_shape[0],
                                                      projection_shape[1], output_shape[0],
                                                      output_shape[1], p=projection_prob,
                                                      output_sparsity_mask=output_sparsity_mask)
        connections = c_helper.grow_synapses(
            input_ids=self.get_lookup_neuron_ids()[::n_detectors_in_group * n_lut_channels] + 1,
            output_ids=self.get_output_neuron_ids().reshape(output_shape) + 1, seed=random_seed)
        connections = repeat_connections_incrementing_source(connections,
                                                             n_lut_channels * n_detectors_in_group)
        self.add_lookup_connections(chunk_of_connections=connections, ids_shift=-1,
                                    random_seed=random_seed)
        self.compile_lut()

    def input_shape(self):
        return self._input_shape

    def output_shape(self):
        return self._output_shape

    def detectors_shape(self):
        return (self._n_detector_groups, self._n_detectors_in_group)

    def export_weights(self):
        n_synapses = self.n_synapses()
        source_ids = torch.zeros([n_synapses], dtype=torch.int32)
        target_ids = torch.zeros([n_synapses], dtype=torch.int32)
        weights = torch.zeros([n_synapses], dtype=torch.float32)
        self._export_synapses(self.get_lookup_neuron_ids(), source_ids, weights, target_ids)
        order = torch.argsort(source_ids, stable=True, descending=False)
        order = order[torch.argsort(target_ids[order], stable=True, descending=False)]
        return weights[order], source_ids[order], target_ids[order]

    def __repr__(self):
        return (f'ProjectionLUTLayer(input_shape={self.input_shape()}, output_shape={self.output_shape()}, '
                f'n_detectors={self._n_detectors}, n_anchors_per_detector={self.n_anchors_per_detector()})')
