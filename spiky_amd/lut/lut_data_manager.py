"""LUTDataManagerF / LUTDataManagerI: the drop-in replacement of the reference's
pybind11 classes (spiky_cuda/lut/lut.cu:1476-1656), implemented over the C ABI
of libspiky_lut.so (include/spiky_lut.h).

Same constructor, same method names, same argument order and defaults, same
tensor conventions (flat, contiguous, fp32 "real" / int32 / int64 stream
handles; checkTensor, spiky_cuda/misc/misc.cpp:217-277) and the same exception
types (ValueError for semantic errors, RuntimeError for tensor/device errors).

Differences, all deliberate:
  * Compute runs only on HIP devices.  A manager on the CPU (device -1) accepts
    every build-time call but its forward/backward raise RuntimeError: there is
    no CPU fallback in the product.
  * Kernels run on the caller's current HIP stream (or on r_stream_handles[0],
    ordered after the current stream).  Nothing synchronises the host.
  * Sparse connectivity is kept as this library's CSR (lookup neuron ->
    ascending output ids), not as the reference's ConnectionsManager layout;
    weights of a sparse layer are one fp32 per synapse in that CSR order.
"""
import ctypes

import numpy as np
import torch

from .. import _native
from ..util.chunk_of_connections import parse_connections

EPS = 0.00000000000000001          # spiky_cuda/misc/misc.h:90
DENOMINATOR32 = 0x000FFFFF         # spiky_cuda/misc/misc.h:98


def check_tensor(t, name, real_or_int, device, sizeof_int=4):
    """checkTensor (spiky_cuda/misc/misc.cpp:217-277)."""
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"tensor {name} must be a torch.Tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"tensor {name} must be contiguous")
    if t.dim() != 1 or t.stride(0) != 1:
        raise RuntimeError(f"tensor {name} must be flat and has stride = 1")
    if real_or_int:
        if t.dtype != torch.float32:
            raise RuntimeError(
                f"tensor {name} must have real data type (float or double depending on build)")
    else:
        if sizeof_int == 1 and t.dtype != torch.int8:
            raise RuntimeError(f"tensor {name} must have dtype int8")
        if sizeof_int == 4 and t.dtype != torch.int32:
            raise RuntimeError(f"tensor {name} must have dtype int32")
        if sizeof_int == 8 and t.dtype != torch.int64:
            raise RuntimeError(f"tensor {name} must have dtype int64")
    if t.layout != torch.strided:
        raise RuntimeError(f"tensor {name} must be strided")
    if device == -1:
        if t.device.type != "cpu":
            raise RuntimeError(f"tensor {name} must be on CPU")
    else:
        if t.device.type != "cuda":
            raise RuntimeError(f"tensor {name} must be on CUDA")
        if t.device.index != device:
            raise RuntimeError(f"tensor {name} must be on CUDA device {device}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require_numel(t, n, name):
    if t.numel() < n:
        raise ValueError(f"{name} has {t.numel()} elements, expected at least {n}")


class _LUTDataManagerBase:
    _SUMMATION = "float32"

    def __init__(self, n_inputs, n_outputs, n_detectors, n_anchors_per_detector, sequence_length,
                 positional_dim, initial_synapse_capacity, forward_group_size,
                 backward_group_size, int_rescaler=None):
        self._args = (n_inputs, n_outputs, n_detectors, n_anchors_per_detector, sequence_length,
                      positional_dim, initial_synapse_capacity, forward_group_size,
                      backward_group_size, int_rescaler)
        for v, nm in ((n_inputs, "n_inputs"), (n_outputs, "n_outputs"),
                      (n_detectors, "n_detectors"), (n_anchors_per_detector, "n_anchors_per_detector"),
                      (sequence_length, "sequence_length"), (forward_group_size, "forward_group_size"),
                      (backward_group_size, "backward_group_size"), (positional_dim, "positional_dim")):
            if int(v) < 0:
                raise TypeError(f"{nm} must be a non-negative integer")
        self._n_inputs = int(n_inputs)
        self._n_outputs = int(n_outputs)
        self._n_detectors = int(n_detectors)
        self._n_anchors = int(n_anchors_per_detector)
        self._sequence_length = int(sequence_length)
        self._positional_dim = int(positional_dim)
        self._forward_group_size = int(forward_group_size)
        self._backward_group_size = int(backward_group_size)
        self._int_mode = int_rescaler is not None
        self._int_rescaler = float(int_rescaler) if int_rescaler is not None else 0.0
        self._device = -1
        handle = ctypes.c_void_p()
        L = _native.lib()
        _native.check(L.spiky_lut_create(
            self._n_inputs, self._n_outputs, self._n_detectors, self._n_anchors,
            self._sequence_length, self._positional_dim, int(initial_synapse_capacity),
            self._forward_group_size, self._backward_group_size, int(self._int_mode),
            self._int_rescaler, ctypes.byref(handle)))
        self._h = handle
        self._n_lookup = int(L.spiky_lut_n_lookup_neurons(self._h))
        self._metas = []
        self._fully_connected = None
        # detector connectivity (build time): target detector -> list of input ids
        self._detector_inputs = None
        self._max_inputs_per_detector = None
        # lookup connectivity (build time): lookup neuron -> list of output ids
        self._lookup_targets = None
        self._n_synapses = 0
        self._compiled = False

    # ---------------------------------------------------------------- pickling
    def __getstate__(self):
        """pickle_lut_neuron_manager (lut.cu:1409-1438): only a manager on the
        CPU serialises.  The state is this object's build-time record (sizes,
        synapse metas, connectivity); the native manager is rebuilt from it."""
        if self._device != -1:
            raise RuntimeError("net must be on CPU before serialization")
        return {k: v for k, v in self.__dict__.items() if k != "_h"}

    def __setstate__(self, state):
        """unpickle_lut_neuron_manager (lut.cu:1440-1473)."""
        self.__dict__.update(state)
        L = _native.lib()
        handle = ctypes.c_void_p()
        _native.check(L.spiky_lut_create(
            self._n_inputs, self._n_outputs, self._n_detectors, self._n_anchors,
            self._sequence_length, self._positional_dim, int(self._args[6]),
            self._forward_group_size, self._backward_group_size, int(self._int_mode),
            self._int_rescaler, ctypes.byref(handle)))
        self._h = handle
        out = ctypes.c_uint32()
        for meta in self._metas:
            _native.check(L.spiky_lut_register_synapse_meta(self._h, *meta, ctypes.byref(out)))
        if self._fully_connected is not None:
            _native.check(L.spiky_lut_initialize_neurons(self._h, int(self._fully_connected)))
        if getattr(self, "_ordered_sums", False):
            _native.check(L.spiky_lut_set_ordered_sums(self._h, 1))
        if self._compiled and not self._fully_connected:
            offs, tg = self._csr
            _native.check(L.spiky_lut_set_sparse_connectivity(
                self._h, offs.ctypes.data_as(ctypes.c_void_p),
                tg.ctypes.data_as(ctypes.c_void_p) if tg.size else None, int(tg.size)))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _native.lib().spiky_lut_destroy(h)
            except Exception:
                pass
            self._h = None

    # ---------------------------------------------------------------- scalars
    def get_smallest_distinguishable_fraction(self):
        if self._int_mode:
            return (1.0 / DENOMINATOR32) / self._int_rescaler
        return 0.0

    def get_epsilon(self):
        return EPS

    def get_summations_data_type(self):
        return self._SUMMATION

    def get_number_of_inputs(self):
        return self._n_inputs

    def get_number_of_outputs(self):
        return self._n_outputs

    def get_number_of_detectors(self):
        return self._n_detectors

    def get_number_of_lookup_neurons(self):
        return self._n_lookup

    def get_number_of_anchors_per_detector(self):
        return self._n_anchors

    def get_number_of_synapses(self):
        return self._n_synapses

    def get_weights_dimension(self):
        if self._fully_connected:
            return self._n_lookup * self._n_outputs
        return self._n_synapses

    def get_max_forward_groups_per_neuron(self):
        return int(_native.lib().spiky_lut_max_forward_groups_per_neuron(self._h))

    # ---------------------------------------------------------------- build time
    def register_synapse_meta(self, learning_rate, min_synaptic_weight, max_synaptic_weight,
                              initial_noise_level, initial_weight):
        out = ctypes.c_uint32()
        _native.check(_native.lib().spiky_lut_register_synapse_meta(
            self._h, float(learning_rate), float(min_synaptic_weight), float(max_synaptic_weight),
            float(initial_noise_level), float(initial_weight), ctypes.byref(out)))
        meta = (float(learning_rate), float(min_synaptic_weight), float(max_synaptic_weight),
                float(initial_noise_level), float(initial_weight))
        if out.value == len(self._metas):
            self._metas.append(meta)
        return int(out.value)

    def initialize_neurons(self, is_fully_connected):
        _native.check(_native.lib().spiky_lut_initialize_neurons(self._h, int(bool(is_fully_connected))))
        self._fully_connected = bool(is_fully_connected)
        if not self._fully_connected:
            self._lookup_targets = {}

    def add_detector_connections(self, connections_buffer, single_input_group_size, ids_shift,
                                 random_seed=None):
        """Detector input lists from a ChunkOfConnections buffer (lut.cu:332-430):
        sources are input neurons [0, n_inputs), targets detector neurons
        [n_inputs, n_inputs + n_detectors) after ids_shift.  The lists are built on
        the host, so the buffer may live on the host or on the manager's device."""
        check_tensor(connections_buffer, "connections_buffer", False,
                     -1 if connections_buffer.device.type == "cpu" else self._device, 4)
        src, tgt = parse_connections(connections_buffer, single_input_group_size, ids_shift)
        det = tgt - self._n_inputs
        ok = (src >= 0) & (src < self._n_inputs) & (det >= 0) & (det < self._n_detectors)
        if not np.all(ok):
            raise ValueError("detector connection ids out of range")
        if self._detector_inputs is None:
            self._detector_inputs = [[] for _ in range(self._n_detectors)]
        for d, s in zip(det.tolist(), src.tolist()):
            self._detector_inputs[d].append(s)

    def finalize_detector_connections(self):
        """Sorts every detector's input list ascending (the CPU order of the
        reference's backward synapse list) and returns the largest list size."""
        if self._detector_inputs is None:
            raise ValueError(
                "detector connections manager not initialized, add detector connections first")
        self._detector_inputs = [sorted(set(v)) for v in self._detector_inputs]
        self._max_inputs_per_detector = max((len(v) for v in self._detector_inputs), default=0)
        return self._max_inputs_per_detector

    def initialize_detectors(self, encoded_pairs_permutations, max_n_inputs_per_detector,
                             detector_anchors, compact_mode):
        """prepare_detectors(_compact) (lut_compile_time_kernels_logic.proto:1-125).
        The decode runs on the host, so both tensors may live on the host or on
        the manager's device."""
        for t, nm in ((encoded_pairs_permutations, "encoded_pairs_permutations"),
                      (detector_anchors, "detector_anchors")):
            check_tensor(t, nm, False, -1 if t.device.type == "cpu" else self._device, 4)
        if self._detector_inputs is None:
            raise ValueError("detector_connections_manager not initialized")
        n = int(max_n_inputs_per_detector)
        per = n if compact_mode else n * (n - 1)
        if per <= 0 or encoded_pairs_permutations.numel() % per != 0:
            raise ValueError("(encoded_pairs_permutations.numel() % max_n_inputs_per_detector) != 0")
        if encoded_pairs_permutations.numel() // per != self._n_detectors:
            raise ValueError("provided_n_detectors != this->n_detectors")
        if detector_anchors.numel() != self._n_detectors * self._n_anchors * 2:
            raise ValueError("detector_anchors.numel() != n_detectors * n_anchors_per_detector * 2")
        lists = self._detector_inputs
        offsets = np.zeros(self._n_detectors + 1, dtype=np.int64)
        offsets[1:] = np.cumsum([len(v) for v in lists])
        ids = np.array([i for v in lists for i in v], dtype=np.int32)
        codes = encoded_pairs_permutations.detach().cpu().numpy().view(np.uint32)
        out = np.zeros(self._n_detectors * self._n_anchors * 2, dtype=np.int32)
        if compact_mode:
            if per < self._n_anchors:
                raise ValueError("max_n_inputs_per_detector < n_anchors_per_detector")
            _native.check(_native.lib().spiky_lut_decode_anchors_compact(
                codes.ctypes.data_as(ctypes.c_void_p), self._n_detectors, per, self._n_anchors,
                offsets.ctypes.data_as(ctypes.c_void_p),
                ids.ctypes.data_as(ctypes.c_void_p) if ids.size else None,
                out.ctypes.data_as(ctypes.c_void_p)))
        else:
            out = _decode_anchors_permutation(codes, per, self._n_anchors, offsets, ids,
                                              self._n_detectors)
        detector_anchors.copy_(torch.from_numpy(out).to(detector_anchors.device))
        # the reference drops the detector connectivity after this call (lut.cu:553-557)
        self._detector_inputs = None

    def detector_input_lists(self):
        return self._detector_inputs

    def add_lookup_connections(self, connections_buffer, single_input_group_size, ids_shift,
                               random_seed=None):
        """Lookup neuron -> output synapses from a ChunkOfConnections buffer
        (lut.cu:560-578): sources are lookup neurons [0, n_lookup), targets
        output neurons [n_lookup, n_lookup + n_outputs) after ids_shift.  Built on
        the host: the buffer may live on the host or on the manager's device."""
        if self._fully_connected:
            raise ValueError("can't add lookup connections in fully connected mode")
        if self._fully_connected is None:
            raise ValueError("neurons are not initialized (call initialize_neurons first)")
        check_tensor(connections_buffer, "connections_buffer", False,
                     -1 if connections_buffer.device.type == "cpu" else self._device, 4)
        src, tgt = parse_connections(connections_buffer, single_input_group_size, ids_shift)
        out = tgt - self._n_lookup
        ok = (src >= 0) & (src < self._n_lookup) & (out >= 0) & (out < self._n_outputs)
        if not np.all(ok):
            raise ValueError("lookup connection ids out of range")
        added = 0
        for s, o in zip(src.tolist(), out.tolist()):
            lst = self._lookup_targets.setdefault(s, set())
            if o not in lst:
                lst.add(o)
                added += 1
        self._n_synapses += added

    def set_lookup_connectivity(self, syn_offsets, syn_targets):
        """Install a lookup-neuron CSR directly (this library's builder path)."""
        if self._fully_connected is not False:
            raise ValueError("can't add lookup connections in fully connected mode")
        offs = np.ascontiguousarray(syn_offsets, dtype=np.int64)
        tg = np.ascontiguousarray(syn_targets, dtype=np.int32)
        if offs.size != self._n_lookup + 1:
            raise ValueError("syn_offsets must have n_lookup_neurons + 1 entries")
        self._csr = (offs, tg)
        self._n_synapses = int(tg.size)
        self._lookup_targets = None

    def compile(self, only_trainable_backwards, weights, random_seed=None):
        """Finalises sparse connectivity (lut.cu:580-627): weights get
        initial_weight + initial_noise_level * U[0,1) per synapse, clipped to
        [min_weight, max_weight] (torch RNG, seeded by random_seed if given)."""
        if self._fully_connected:
            raise ValueError("nothing to compile in fully connected mode")
        if random_seed is not None and int(random_seed) == 0:
            raise ValueError("random_seed should be greater than 0")
        if self._fully_connected is None:
            raise ValueError("neurons are not initialized (call initialize_neurons first)")
        check_tensor(weights, "weights", True, self._device)
        if self._lookup_targets is not None:
            counts = np.zeros(self._n_lookup, dtype=np.int64)
            for s, lst in self._lookup_targets.items():
                counts[s] = len(lst)
            offs = np.zeros(self._n_lookup + 1, dtype=np.int64)
            offs[1:] = np.cumsum(counts)
            tg = np.zeros(int(offs[-1]), dtype=np.int32)
            for s, lst in self._lookup_targets.items():
                tg[offs[s]:offs[s + 1]] = sorted(lst)
            self._csr = (offs, tg)
            self._lookup_targets = None
        offs, tg = self._csr
        if weights.numel() != tg.size:
            raise ValueError("wrong weights.numel()")
        _native.check(_native.lib().spiky_lut_set_sparse_connectivity(
            self._h, offs.ctypes.data_as(ctypes.c_void_p),
            tg.ctypes.data_as(ctypes.c_void_p) if tg.size else None, int(tg.size)))
        lr, mn, mx, noise, init = self._metas[0]
        g = torch.Generator(device="cpu")
        if random_seed is not None:
            g.manual_seed(int(random_seed))
        w = torch.rand(tg.size, generator=g if random_seed is not None else None)
        w = (w * noise + init).clamp_(mn, mx)
        weights.copy_(w.to(weights.device))
        self._compiled = True

    def lookup_connectivity(self):
        """(syn_offsets int64 [n_lookup+1], syn_targets int32) of a compiled sparse manager."""
        return getattr(self, "_csr", None)

    def set_ordered_sums(self, ordered):
        """True: the fp32 forward commits one fp32 value per block of
        backward_group_size tables in ascending block order, bit-identical to
        the reference CPU path (lut_runtime_kernels_logic.proto:1214-1299).
        False (default): large batches sum several blocks in fp64 before one
        commit, within the fp32 tolerance of the reference GPU path's
        unordered atomics.  No effect on int32 summation."""
        self._ordered_sums = bool(ordered)
        _native.check(_native.lib().spiky_lut_set_ordered_sums(self._h, int(self._ordered_sums)))

    def to_device(self, device):
        self._device = int(device)

    # ---------------------------------------------------------------- runtime
    def _launch(self, r_stream_handles, call):
        """Runs call(stream) on the manager's device and checks its status.

        Without handles the kernels go on torch's current stream.  With
        handles they go on r_stream_handles[0], which first waits for the
        current stream; afterwards the current stream waits for it, so a
        caller that reads the outputs (or frees the inputs) on the current
        stream is ordered after the kernels, and calls on different handles
        never overlap on the manager's scratch memory.  The reference makes
        the same guarantee by synchronising the device
        (lut_runtime.cu:99,244,423)."""
        self._require_device()
        if r_stream_handles is not None:
            check_tensor(r_stream_handles, "r_stream_handles", False, -1, 8)
            if r_stream_handles.numel() < 3:
                raise ValueError("r_stream_handles must have at least 3 elements")
        dev = torch.device("cuda", self._device)
        with torch.cuda.device(dev):
            cur = torch.cuda.current_stream(dev)
            if r_stream_handles is None:
                _native.check(call(ctypes.c_void_p(cur.cuda_stream)))
                return
            h = int(r_stream_handles[0].item())
            ext = torch.cuda.ExternalStream(h, device=dev)
            ext.wait_stream(cur)
            try:
                _native.check(call(ctypes.c_void_p(h)))
            finally:
                cur.wait_stream(ext)

    def _require_device(self):
        if self._device < 0:
            raise RuntimeError(
                "spiky_amd runs the LUT kernels on HIP devices only; move the layer to a GPU")

    def forward_step(self, r_weights, batch_size, r_input, r_detector_anchors, w_output,
                     w_lookup_indices, cmp_eps=0.0, r_stream_handles=None,
                     w_min_anchor_deltas=None, w_min_anchor_delta_indices=None):
        """lut.cu:629-716 -> lut_runtime.cu:76-211."""
        dev = self._device
        check_tensor(r_weights, "r_weights", True, dev)
        check_tensor(r_input, "r_input", True, dev)
        check_tensor(r_detector_anchors, "r_detector_anchors", False, dev, 4)
        check_tensor(w_output, "w_output", True, dev)
        check_tensor(w_lookup_indices, "w_lookup_indices", False, dev, 4)
        if w_min_anchor_deltas is not None:
            check_tensor(w_min_anchor_deltas, "w_min_anchor_deltas", True, dev)
        if w_min_anchor_delta_indices is not None:
            check_tensor(w_min_anchor_delta_indices, "w_min_anchor_delta_indices", False, dev, 4)
        if batch_size == 0:
            raise ValueError("batch_size == 0")
        B = int(batch_size)
        _require_numel(r_weights, self.get_weights_dimension(), "r_weights")
        _require_numel(r_input, B * self._n_inputs, "r_input")
        _require_numel(r_detector_anchors, self._n_detectors * self._n_anchors * 2, "r_detector_anchors")
        _require_numel(w_output, B * self._n_outputs, "w_output")
        _require_numel(w_lookup_indices, B * self._n_detectors, "w_lookup_indices")
        if w_min_anchor_deltas is not None:
            _require_numel(w_min_anchor_deltas, B * self._n_detectors, "w_min_anchor_deltas")
        if w_min_anchor_delta_indices is not None:
            _require_numel(w_min_anchor_delta_indices, B * self._n_detectors, "w_min_anchor_delta_indices")
        self._launch(r_stream_handles, lambda st: _native.lib().spiky_lut_forward_step(
            self._h, _ptr(r_weights), B, _ptr(r_input), _ptr(r_detector_anchors),
            _ptr(w_output), _ptr(w_lookup_indices), float(cmp_eps), _ptr(w_min_anchor_deltas),
            _ptr(w_min_anchor_delta_indices), st))

    def forward_step_i8(self, r_weights_q8, r_scales, batch_size, r_input, r_detector_anchors,
                        w_output, w_lookup_indices, cmp_eps=0.0, r_stream_handles=None,
                        w_min_anchor_deltas=None, w_min_anchor_delta_indices=None):
        """forward_step over int8 tables with one fp32 scale per detector
        (weight = scale[t] * q); fully connected managers only."""
        dev = self._device
        check_tensor(r_weights_q8, "r_weights_q8", False, dev, 1)
        check_tensor(r_scales, "r_scales", True, dev)
        check_tensor(r_input, "r_input", True, dev)
        check_tensor(r_detector_anchors, "r_detector_anchors", False, dev, 4)
        check_tensor(w_output, "w_output", True, dev)
        check_tensor(w_lookup_indices, "w_lookup_indices", False, dev, 4)
        if w_min_anchor_deltas is not None:
            check_tensor(w_min_anchor_deltas, "w_min_anchor_deltas", True, dev)
        if w_min_anchor_delta_indices is not None:
            check_tensor(w_min_anchor_delta_indices, "w_min_anchor_delta_indices", False, dev, 4)
        if batch_size == 0:
            raise ValueError("batch_size == 0")
        B = int(batch_size)
        _require_numel(r_weights_q8, self._n_lookup * self._n_outputs, "r_weights_q8")
        _require_numel(r_scales, self._n_detectors, "r_scales")
        _require_numel(r_input, B * self._n_inputs, "r_input")
        _require_numel(r_detector_anchors, self._n_detectors * self._n_anchors * 2, "r_detector_anchors")
        _require_numel(w_output, B * self._n_outputs, "w_output")
        _require_numel(w_lookup_indices, B * self._n_detectors, "w_lookup_indices")
        if w_min_anchor_deltas is not None:
            _require_numel(w_min_anchor_deltas, B * self._n_detectors, "w_min_anchor_deltas")
        if w_min_anchor_delta_indices is not None:
            _require_numel(w_min_anchor_delta_indices, B * self._n_detectors, "w_min_anchor_delta_indices")
        self._launch(r_stream_handles, lambda st: _native.lib().spiky_lut_forward_step_i8(
            self._h, _ptr(r_weights_q8), _ptr(r_scales), B, _ptr(r_input),
            _ptr(r_detector_anchors), _ptr(w_output), _ptr(w_lookup_indices), float(cmp_eps),
            _ptr(w_min_anchor_deltas), _ptr(w_min_anchor_delta_indices), st))

    def backward_backprop(self, r_weights, batch_size, r_output_gradients, r_detector_anchors,
                          r_lookup_indices, r_min_anchor_deltas, r_min_anchor_delta_indices,
                          w_input_gradients, external_lr, w_weights_gradients=None,
                          r_stream_handles=None, overwrite_weights_gradients=False):
        """lut.cu:1030-1088 -> lut_runtime.cu:213-397.  The extra keyword
        overwrite_weights_gradients=True lets the kernel overwrite
        w_weights_gradients instead of accumulating into it (no zero-fill needed)."""
        if batch_size == 0:
            raise ValueError("batch_size == 0")
        dev = self._device
        check_tensor(r_weights, "r_weights", True, dev)
        check_tensor(w_input_gradients, "w_input_gradients", True, dev)
        check_tensor(r_output_gradients, "r_output_gradients", True, dev)
        check_tensor(r_detector_anchors, "r_detector_anchors", False, dev, 4)
        check_tensor(r_lookup_indices, "r_lookup_indices", False, dev, 4)
        check_tensor(r_min_anchor_deltas, "r_min_anchor_deltas", True, dev)
        check_tensor(r_min_anchor_delta_indices, "r_min_anchor_delta_indices", False, dev, 4)
        if w_weights_gradients is not None:
            check_tensor(w_weights_gradients, "w_weights_gradients", True, dev)
        B = int(batch_size)
        _require_numel(r_weights, self.get_weights_dimension(), "r_weights")
        _require_numel(r_output_gradients, B * self._n_outputs, "r_output_gradients")
        _require_numel(r_detector_anchors, self._n_detectors * self._n_anchors * 2, "r_detector_anchors")
        _require_numel(w_input_gradients, B * self._n_inputs, "w_input_gradients")
        for t, nm in ((r_lookup_indices, "r_lookup_indices"), (r_min_anchor_deltas, "r_min_anchor_deltas"),
                      (r_min_anchor_delta_indices, "r_min_anchor_delta_indices")):
            _require_numel(t, B * self._n_detectors, nm)
        if w_weights_gradients is not None:
            _require_numel(w_weights_gradients, self.get_weights_dimension(), "w_weights_gradients")
        self._launch(r_stream_handles, lambda st: _native.lib().spiky_lut_backward_backprop(
            self._h, _ptr(r_weights), B, _ptr(r_output_gradients), _ptr(r_detector_anchors),
            _ptr(r_lookup_indices), _ptr(r_min_anchor_deltas), _ptr(r_min_anchor_delta_indices),
            _ptr(w_input_gradients), float(external_lr), _ptr(w_weights_gradients),
            int(bool(overwrite_weights_gradients)), st))

    # ---------------------------------------------------------------- sequence-concat mode
    def forward_step_concat(self, r_weights, batch_size, r_input, r_detector_anchors, w_output,
                            w_lookup_indices, cmp_eps, r_positional_embeddings,
                            w_positional_lookup_indices, w_min_anchor_deltas=None,
                            w_min_anchor_delta_indices=None, w_positional_min_deltas=None,
                            w_positional_min_delta_indices=None, r_stream_handles=None):
        """lut.cu pybind 1556-1575 -> lut_runtime.cu:399-593.  Input [B][S][I];
        lookup indices / min deltas [B][S][T]; positional ones [(S-1)][T]."""
        if batch_size == 0:
            raise ValueError("batch_size == 0")
        dev = self._device
        S = self._sequence_length
        if S <= 1:
            raise ValueError("forward_step_concat should only be called when sequence_length > 1")
        check_tensor(r_weights, "r_weights", True, dev)
        check_tensor(r_input, "r_input", True, dev)
        check_tensor(r_detector_anchors, "r_detector_anchors", False, dev, 4)
        check_tensor(w_output, "w_output", True, dev)
        check_tensor(w_lookup_indices, "w_lookup_indices", False, dev, 4)
        for t, nm, real in ((w_min_anchor_deltas, "w_min_anchor_deltas", True),
                            (w_min_anchor_delta_indices, "w_min_anchor_delta_indices", False),
                            (r_positional_embeddings, "r_positional_embeddings", True),
                            (w_positional_lookup_indices, "w_positional_lookup_indices", False),
                            (w_positional_min_deltas, "w_positional_min_deltas", True),
                            (w_positional_min_delta_indices, "w_positional_min_delta_indices", False)):
            if t is not None:
                check_tensor(t, nm, real, dev)
        B, T, P = int(batch_size), self._n_detectors, self._positional_dim
        _require_numel(r_weights, self.get_weights_dimension(), "r_weights")
        _require_numel(r_input, B * S * self._n_inputs, "r_input")
        _require_numel(r_detector_anchors, T * self._n_anchors * 2, "r_detector_anchors")
        _require_numel(w_output, B * S * self._n_outputs, "w_output")
        _require_numel(w_lookup_indices, B * S * T, "w_lookup_indices")
        for t, nm in ((w_min_anchor_deltas, "w_min_anchor_deltas"),
                      (w_min_anchor_delta_indices, "w_min_anchor_delta_indices")):
            if t is not None:
                _require_numel(t, B * S * T, nm)
        if P > 0:
            for t, nm in ((w_positional_min_deltas, "w_positional_min_deltas"),
                          (w_positional_min_delta_indices, "w_positional_min_delta_indices")):
                if t is not None:
                    _require_numel(t, (S - 1) * T, nm)
            if r_positional_embeddings is None or w_positional_lookup_indices is None:
                raise ValueError("positional embeddings and positional lookup indices must be "
                                 "provided when positional_dim > 0")
            _require_numel(r_positional_embeddings, (S - 1) * T * P, "r_positional_embeddings")
            _require_numel(w_positional_lookup_indices, (S - 1) * T, "w_positional_lookup_indices")
        self._launch(r_stream_handles, lambda st: _native.lib().spiky_lut_forward_step_concat(
            self._h, _ptr(r_weights), B, _ptr(r_input), _ptr(r_detector_anchors), _ptr(w_output),
            _ptr(w_lookup_indices), float(cmp_eps), _ptr(r_positional_embeddings if P > 0 else None),
            _ptr(w_positional_lookup_indices if P > 0 else None), _ptr(w_min_anchor_deltas),
            _ptr(w_min_anchor_delta_indices), _ptr(w_positional_min_deltas if P > 0 else None),
            _ptr(w_positional_min_delta_indices if P > 0 else None), st))

    def backward_backprop_concat(self, r_weights, batch_size, r_output_gradients, r_detector_anchors,
                                 r_lookup_indices, r_min_anchor_deltas, r_min_anchor_delta_indices,
                                 w_input_gradients, external_lr, r_positional_lookup_indices=None,
                                 r_positional_min_deltas=None, r_positional_min_delta_indices=None,
                                 w_positional_embeddings_gradients=None, w_weights_gradients=None,
                                 r_stream_handles=None, overwrite_weights_gradients=False):
        """lut.cu pybind 1620-1636 -> lut_runtime.cu:595-850."""
        if batch_size == 0:
            raise ValueError("batch_size == 0")
        dev = self._device
        S = self._sequence_length
        if S <= 1:
            raise ValueError("backward_backprop_concat should only be called when sequence_length > 1")
        for t, nm, real in ((r_weights, "r_weights", True), (r_output_gradients, "r_output_gradients", True),
                            (r_detector_anchors, "r_detector_anchors", False),
                            (r_lookup_indices, "r_lookup_indices", False),
                            (r_min_anchor_deltas, "r_min_anchor_deltas", True),
                            (r_min_anchor_delta_indices, "r_min_anchor_delta_indices", False),
                            (w_input_gradients, "w_input_gradients", True)):
            check_tensor(t, nm, real, dev)
        for t, nm, real in ((r_positional_lookup_indices, "r_positional_lookup_indices", False),
                            (r_positional_min_deltas, "r_positional_min_deltas", True),
                            (r_positional_min_delta_indices, "r_positional_min_delta_indices", False),
                            (w_positional_embeddings_gradients, "w_positional_embeddings_gradients", True),
                            (w_weights_gradients, "w_weights_gradients", True)):
            if t is not None:
                check_tensor(t, nm, real, dev)
        B, T, P = int(batch_size), self._n_detectors, self._positional_dim
        _require_numel(r_weights, self.get_weights_dimension(), "r_weights")
        _require_numel(r_output_gradients, B * S * self._n_outputs, "r_output_gradients")
        _require_numel(r_detector_anchors, T * self._n_anchors * 2, "r_detector_anchors")
        _require_numel(w_input_gradients, B * S * self._n_inputs, "w_input_gradients")
        for t, nm in ((r_lookup_indices, "r_lookup_indices"), (r_min_anchor_deltas, "r_min_anchor_deltas"),
                      (r_min_anchor_delta_indices, "r_min_anchor_delta_indices")):
            _require_numel(t, B * S * T, nm)
        if P > 0:
            for t, nm in ((r_positional_lookup_indices, "r_positional_lookup_indices"),
                          (r_positional_min_deltas, "r_positional_min_deltas"),
                          (r_positional_min_delta_indices, "r_positional_min_delta_indices")):
                if t is None:
                    raise ValueError(f"{nm} must be provided when positional_dim > 0")
                _require_numel(t, (S - 1) * T, nm)
            if w_positional_embeddings_gradients is None:
                raise ValueError("w_positional_embeddings_gradients must be provided when positional_dim > 0")
            _require_numel(w_positional_embeddings_gradients, (S - 1) * T * P,
                           "w_positional_embeddings_gradients")
        if w_weights_gradients is not None:
            _require_numel(w_weights_gradients, self.get_weights_dimension(), "w_weights_gradients")
        self._launch(r_stream_handles, lambda st: _native.lib().spiky_lut_backward_backprop_concat(
            self._h, _ptr(r_weights), B, _ptr(r_output_gradients), _ptr(r_detector_anchors),
            _ptr(r_lookup_indices), _ptr(r_min_anchor_deltas), _ptr(r_min_anchor_delta_indices),
            _ptr(w_input_gradients), float(external_lr),
            _ptr(r_positional_lookup_indices if P > 0 else None),
            _ptr(r_positional_min_deltas if P > 0 else None),
            _ptr(r_positional_min_delta_indices if P > 0 else None),
            _ptr(w_positional_embeddings_gradients if P > 0 else None), _ptr(w_weights_gradients),
            int(bool(overwrite_weights_gradients)), st))

    def _product_sizes(self, batch_size, sequence_length, n_inputs_1, n_inputs_2, what):
        if batch_size == 0:
            raise ValueError("batch_size == 0")
        if self._sequence_length != 1:
            raise ValueError(f"{what}: this is an experimental method, this->sequence_length should be "
                             "equal to 1, real length of the sequence is passed as the method parameter")
        if sequence_length == 0:
            raise ValueError("sequence_length == 0")
        return int(batch_size), int(sequence_length), int(n_inputs_1), int(n_inputs_2)

    def forward_step_product(self, r_weights, batch_size, sequence_length, r_input_1, r_input_2,
                             r_detector_anchors, w_output, n_inputs_1, n_inputs_2, sliced_mode=False,
                             cmp_eps=0.0, r_positional_embeddings=None, r_stream_handles=None):
        """lut.cu:847-943 -> lut_runtime.cu:852-1049.  The manager has
        sequence_length 1; the real one is the argument.  r_input_1 [B][S][n1],
        r_input_2 [B][S][n2], w_output [B][S][O] summed into, positional
        embeddings [(S-1)][T][pd]."""
        dev = self._device
        B, S, n1, n2 = self._product_sizes(batch_size, sequence_length, n_inputs_1, n_inputs_2,
                                           "forward_step_product")
        check_tensor(r_weights, "r_weights", True, dev)
        check_tensor(r_input_1, "r_input_1", True, dev)
        check_tensor(r_input_2, "r_input_2", True, dev)
        check_tensor(r_detector_anchors, "r_detector_anchors", False, dev, 4)
        check_tensor(w_output, "w_output", True, dev)
        if r_positional_embeddings is not None:
            check_tensor(r_positional_embeddings, "r_positional_embeddings", True, dev)
        T, P = self._n_detectors, self._positional_dim
        _require_numel(r_weights, self.get_weights_dimension(), "r_weights")
        _require_numel(r_input_1, B * S * n1, "r_input_1")
        _require_numel(r_input_2, B * S * n2, "r_input_2")
        _require_numel(r_detector_anchors, T * self._n_anchors * 2, "r_detector_anchors")
        _require_numel(w_output, B * S * self._n_outputs, "w_output")
        if P > 0:
            if r_positional_embeddings is None:
                raise ValueError("r_positional_embeddings must be provided when positional_dim > 0")
            _require_numel(r_positional_embeddings, (S - 1) * T * P, "r_positional_embeddings")
        self._launch(r_stream_handles, lambda st: _native.lib().spiky_lut_forward_step_product(
            self._h, _ptr(r_weights), B, S, _ptr(r_input_1), _ptr(r_input_2),
            _ptr(r_detector_anchors), _ptr(w_output), n1, n2, int(bool(sliced_mode)),
            float(cmp_eps), _ptr(r_positional_embeddings if P > 0 else None),
            st))

    def backward_backprop_product(self, r_weights, batch_size, sequence_length, r_input_1, r_input_2,
                                  r_detector_anchors, r_output_gradients, w_input_gradients_1,
                                  w_input_gradients_2, external_lr, n_inputs_1, n_inputs_2,
                                  sliced_mode=False, cmp_eps=0.0, w_weights_gradients=None,
                                  r_positional_embeddings=None, w_positional_embeddings_gradients=None,
                                  r_stream_handles=None):
        """lut.cu:945-1039 -> lut_runtime.cu:1051-1456.  The two input
        gradients may be one tensor (the layer's call)."""
        dev = self._device
        B, S, n1, n2 = self._product_sizes(batch_size, sequence_length, n_inputs_1, n_inputs_2,
                                           "backward_backprop_product")
        for t, nm, real in ((r_weights, "r_weights", True), (r_input_1, "r_input_1", True),
                            (r_input_2, "r_input_2", True),
                            (r_detector_anchors, "r_detector_anchors", False),
                            (r_output_gradients, "r_output_gradients", True),
                            (w_input_gradients_1, "w_input_gradients_1", True),
                            (w_input_gradients_2, "w_input_gradients_2", True)):
            check_tensor(t, nm, real, dev)
        for t, nm in ((w_weights_gradients, "w_weights_gradients"),
                      (r_positional_embeddings, "r_positional_embeddings"),
                      (w_positional_embeddings_gradients, "w_positional_embeddings_gradients")):
            if t is not None:
                check_tensor(t, nm, True, dev)
        T, P = self._n_detectors, self._positional_dim
        _require_numel(r_weights, self.get_weights_dimension(), "r_weights")
        _require_numel(r_input_1, B * S * n1, "r_input_1")
        _require_numel(r_input_2, B * S * n2, "r_input_2")
        _require_numel(r_detector_anchors, T * self._n_anchors * 2, "r_detector_anchors")
        _require_numel(r_output_gradients, B * S * self._n_outputs, "r_output_gradients")
        _require_numel(w_input_gradients_1, B * S * n1, "w_input_gradients_1")
        _require_numel(w_input_gradients_2, B * S * n2, "w_input_gradients_2")
        if w_weights_gradients is not None:
            _require_numel(w_weights_gradients, self.get_weights_dimension(), "w_weights_gradients")
        if P > 0:
            if r_positional_embeddings is None or w_positional_embeddings_gradients is None:
                raise ValueError("positional embeddings and their gradients must be provided when "
                                 "positional_dim > 0")
            _require_numel(r_positional_embeddings, (S - 1) * T * P, "r_positional_embeddings")
            _require_numel(w_positional_embeddings_gradients, (S - 1) * T * P,
                           "w_positional_embeddings_gradients")
        self._launch(r_stream_handles, lambda st: _native.lib().spiky_lut_backward_backprop_product(
            self._h, _ptr(r_weights), B, S, _ptr(r_input_1), _ptr(r_input_2),
            _ptr(r_detector_anchors), _ptr(r_output_gradients), _ptr(w_input_gradients_1),
            _ptr(w_input_gradients_2), float(external_lr), n1, n2, int(bool(sliced_mode)),
            float(cmp_eps), _ptr(w_weights_gradients),
            _ptr(r_positional_embeddings if P > 0 else None),
            _ptr(w_positional_embeddings_gradients if P > 0 else None), st))

    # ---------------------------------------------------------------- export
    def count_synapses(self, neuron_indices_to_process):
        """Number of forward synapses of the given lookup neurons."""
        csr = self.lookup_connectivity()
        if csr is None:
            return 0
        offs = csr[0]
        ids = neuron_indices_to_process.detach().cpu().numpy().astype(np.int64)
        return int(np.sum(offs[ids + 1] - offs[ids]))

    def export_synapses(self, weights, neuron_indices_to_process, target_internal_source_indices,
                        target_weights, target_internal_target_indices,
                        target_synapse_meta_indices=None):
        """Writes (source lookup id, weight, target output neuron id) of every
        synapse of the given lookup neurons, in CSR order."""
        csr = self.lookup_connectivity()
        if csr is None:
            raise ValueError("nothing to export")
        offs, tg = csr
        ids = neuron_indices_to_process.detach().cpu().numpy().astype(np.int64)
        sel = np.concatenate([np.arange(offs[i], offs[i + 1]) for i in ids]) if ids.size else \
            np.zeros(0, dtype=np.int64)
        src = np.repeat(ids, offs[ids + 1] - offs[ids]).astype(np.int32)
        w = weights.detach().cpu().numpy()[sel]
        n = sel.size
        target_internal_source_indices[:n] = torch.from_numpy(src).to(target_internal_source_indices.device)
        target_weights[:n] = torch.from_numpy(w).to(target_weights.device)
        target_internal_target_indices[:n] = torch.from_numpy(
            (tg[sel] + self._n_lookup).astype(np.int32)).to(target_internal_target_indices.device)
        if target_synapse_meta_indices is not None:
            target_synapse_meta_indices[:n] = 0
        return n

    # ---------------------------------------------------------------- stats
    def __repr__(self):
        return (f"LUTDataManager(summation type: {self._SUMMATION}; smallest distinguishable "
                f"fraction: {self.get_smallest_distinguishable_fraction()}; n_synapses: "
                f"{self._n_synapses}; n_detectors: {self._n_detectors}; n_lookup_neurons: "
                f"{self._n_lookup}; device: {self._device})")

    def get_memory_stats(self):
        csr = self.lookup_connectivity()
        syn_kb = 0 if csr is None else (csr[0].nbytes + csr[1].nbytes) // 1024
        return (f"synapse metas: 0 KB\nneuron infos: 0 KB\ndetectors: 0 KB\n"
                f"forward main synapses: {syn_kb} KB\nbackward synapses: 0 KB\ndelays info: 0 KB\n")

    def get_profiling_stats(self):
        buf = ctypes.create_string_buffer(1 << 16)
        _native.check(_native.lib().spiky_lut_profiling_stats(self._h, buf, len(buf)))
        return buf.value.decode()

    def reset_profiler(self):
        _native.lib().spiky_lut_reset_profiler(self._h)

    def set_kernel_timing(self, enable):
        """Bracket every kernel launch with HIP events on its stream."""
        _native.check(_native.lib().spiky_lut_set_kernel_timing(self._h, int(bool(enable))))

    def get_kernel_times(self, reset=False):
        """{kernel family: (launches, total GPU ms)} of the timed launches so far
        (waits for the recorded events)."""
        buf = ctypes.create_string_buffer(1 << 16)
        _native.check(_native.lib().spiky_lut_kernel_times(self._h, buf, len(buf), int(bool(reset))))
        res = {}
        for line in buf.value.decode().splitlines():
            name, cnt, ms = line.split()
            res[name] = (int(cnt), float(ms))
        return res

    # ---------------------------------------------------------------- pickle
    def __getstate__(self):
        if self._device != -1:
            raise RuntimeError("net must be on CPU before serialization")
        return {"args": self._args, "metas": self._metas, "fc": self._fully_connected,
                "csr": self.lookup_connectivity(), "n_syn": self._n_synapses}

    def __setstate__(self, st):
        a = st["args"]
        self.__init__(*a[:9], **({} if a[9] is None else {"int_rescaler": a[9]}))
        for m in st["metas"]:
            self.register_synapse_meta(*m)
        if st["fc"] is not None:
            self.initialize_neurons(st["fc"])
        if st["csr"] is not None:
            self.set_lookup_connectivity(*st["csr"])
            offs, tg = st["csr"]
            _native.check(_native.lib().spiky_lut_set_sparse_connectivity(
                self._h, offs.ctypes.data_as(ctypes.c_void_p),
                tg.ctypes.data_as(ctypes.c_void_p) if tg.size else None, int(tg.size)))
            self._compiled = True


def _decode_anchors_permutation(codes, per, n_anchors, offsets, ids, n_detectors):
    """prepare_detectors_logic (lut_compile_time_kernels_logic.proto:1-68):
    walk the permutation, keep codes below n(n-1), pad with -1."""
    out = np.full(n_detectors * n_anchors * 2, -1, dtype=np.int32)
    for i in range(n_detectors):
        n = int(offsets[i + 1] - offsets[i])
        if n <= 1:
            raise ValueError("Some detectors have <= 1 input synapses")
        lst = ids[offsets[i]:offsets[i + 1]]
        maxc = n * (n - 1)
        got = 0
        for c in codes[i * per:(i + 1) * per]:
            if got >= n_anchors:
                break
            c = int(c)
            if c < maxc:
                a1, a2 = divmod(c, n - 1)
                if a2 >= a1:
                    a2 += 1
                out[(i * n_anchors + got) * 2] = lst[a1]
                out[(i * n_anchors + got) * 2 + 1] = lst[a2]
                got += 1
    return out


class LUTDataManagerF(_LUTDataManagerBase):
    """fp32 summation manager (reference LUTDataManagerF)."""
    _SUMMATION = "float32"

    def __init__(self, n_inputs, n_outputs, n_detectors, n_anchors_per_detector, sequence_length,
                 positional_dim, initial_synapse_capacity, forward_group_size, backward_group_size):
        super().__init__(n_inputs, n_outputs, n_detectors, n_anchors_per_detector, sequence_length,
                         positional_dim, initial_synapse_capacity, forward_group_size,
                         backward_group_size, None)


class LUTDataManagerI(_LUTDataManagerBase):
    """int32 fixed-point summation manager (reference LUTDataManagerI,
    spiky_cuda/lut/aux/lut_I.cu:1-2)."""
    _SUMMATION = "int32"

    def __init__(self, n_inputs, n_outputs, n_detectors, n_anchors_per_detector, sequence_length,
                 positional_dim, initial_synapse_capacity, forward_group_size, backward_group_size,
                 int_rescaler):
        super().__init__(n_inputs, n_outputs, n_detectors, n_anchors_per_detector, sequence_length,
                         positional_dim, initial_synapse_capacity, forward_group_size,
                         backward_group_size, int_rescaler)
