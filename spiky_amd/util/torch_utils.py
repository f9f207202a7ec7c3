"""Dense -> sparse (COO) conversion of 32-bit tensors on the device.

Mirror of the reference's ``spiky.util.torch_utils.DenseToSparseConverter``
(src/spiky/util/torch_utils.py:7-125): the same methods, arguments, buffer
rules and error texts, backed by the HIP compaction in
``spiky_amd/csrc/lut_densify.hip`` through the C ABI
(``spiky_count_nonzero32`` / ``spiky_dense_to_sparse32``).

Differences from the reference, both deliberate:

- the output is in ascending index order (the reference orders it only within
  a kernel block), so a COO tensor built from it is truly coalesced;
- ``dense_to_sparse_32`` without ``densify_buffers`` returns the arrays it
  allocated.  The reference passes ``None`` to ``decouple_results`` on that
  path (torch_utils.py:103-107) and raises ``TypeError``; its own test stops
  after the first of its four cases (torch_utils.py:192), which uses buffers.

A word is kept when its 32-bit pattern is non-zero, as in the reference's int4
compare: a float ``-0.0`` is kept.
"""
from typing import Optional, Tuple

import torch

from .. import _native


class DenseToSparseConverter:
    """Converter of dense 1-D 32-bit tensors to (indices, values), reusable
    across calls (reference torch_utils.py:7-22)."""

    def __init__(self, use_new_kernel: bool = True):
        # the reference chooses between two kernels of identical output; one here
        self._use_new_kernel = use_new_kernel
        self._counter_buffer = None
        self._workspace = None
        self._calls = 0

    def __getstate__(self):
        # the counter and workspace are device caches, rebuilt on first use
        st = dict(self.__dict__)
        st["_counter_buffer"] = None
        st["_workspace"] = None
        return st

    def _ensure(self, source):
        dev = source.device
        if self._counter_buffer is None or self._counter_buffer.device != dev:
            self._counter_buffer = torch.zeros(1, dtype=torch.int64, device=dev)
        need = int(_native.lib().spiky_densify32_workspace_bytes(source.numel()))
        if self._workspace is None or self._workspace.device != dev or self._workspace.numel() < need:
            self._workspace = torch.empty(max(need, 8), dtype=torch.uint8, device=dev)

    def count_nonzero(self, source: torch.Tensor) -> int:
        """Number of non-zero 32-bit words of ``source`` (synchronises)."""
        self._check_source(source)
        self._ensure(source)
        stream = torch.cuda.current_stream(source.device).cuda_stream
        _native.check(_native.lib().spiky_count_nonzero32(
            source.data_ptr(), source.numel(), self._workspace.data_ptr(), self._workspace.numel(),
            self._counter_buffer.data_ptr(), stream))
        return int(self._counter_buffer.item())

    @staticmethod
    def _check_source(source):
        # torch_utils.py:59-64
        if source.element_size() != 4:
            raise ValueError(f"source tensor must be 32-bit (element_size == 4), got {source.element_size()}")
        if (source.numel() % 4) != 0:
            raise ValueError(f"source tensor size must be divisable by 4")
        if source.device.type != "cuda":
            raise ValueError("source tensor must be on a GPU device")
        if not source.is_contiguous():
            raise ValueError("source tensor must be contiguous")

    def dense_to_sparse_32(
        self,
        source: torch.Tensor,
        erase_input: bool = False,
        densify_buffers: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
        stream: Optional[torch.cuda.Stream] = None,
        decouple=True
    ) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """Indices (int64) and values of the non-zero words of the 1-D 32-bit
        ``source`` (reference torch_utils.py:35-107); ``(None, None)`` when
        there are none.  ``erase_input`` zeroes the kept words.  With
        ``densify_buffers`` the results go to those tensors (no counting pass
        first) and ``decouple`` returns copies of their used prefix."""
        self._check_source(source)
        self._ensure(source)
        provided_buffers = densify_buffers is not None
        if provided_buffers:
            indices, values = densify_buffers
            if values.dim() != 1 or indices.dim() != 1:
                raise ValueError("densify_buffers tensors must be 1D")
            if values.dtype != source.dtype:
                raise ValueError("densify_buffers values tensor must match source dtype")
            if indices.dtype != torch.int64:
                raise ValueError("densify_buffers indices tensor must be int64")
            if values.device != source.device or indices.device != source.device:
                raise ValueError("densify_buffers tensors must be on the same device as source")
            if not values.is_contiguous() or not indices.is_contiguous():
                raise ValueError("densify_buffers tensors must be contiguous")
            if values.numel() != indices.numel():
                raise ValueError("densify_buffers tensors must have the same length")
            counted = 0
        else:
            assert decouple
            nnz = self.count_nonzero(source)
            if nnz == 0:
                return None, None
            indices = torch.empty(nnz, dtype=torch.int64, device=source.device)
            values = torch.empty(nnz, dtype=source.dtype, device=source.device)
            counted = 1
        handle = stream.cuda_stream if stream is not None else torch.cuda.current_stream(source.device).cuda_stream
        _native.check(_native.lib().spiky_dense_to_sparse32(
            source.data_ptr(), source.numel(), indices.data_ptr(), values.data_ptr(), indices.numel(),
            self._workspace.data_ptr(), self._workspace.numel(), self._counter_buffer.data_ptr(),
            int(bool(erase_input)), counted, handle))
        self._calls += 1
        if decouple:
            if stream is not None:
                stream.synchronize()
            if provided_buffers:
                return self.decouple_results(densify_buffers)
            return indices, values
        return indices, values

    def decouple_results(self, provided_buffers):
        """Copies of the used prefix of the buffers (torch_utils.py:109-116)."""
        indices, values = provided_buffers
        nnz_written = int(self._counter_buffer.item())
        if nnz_written == 0:
            return None, None
        if nnz_written > indices.numel():
            raise ValueError(f"densify_buffers hold {indices.numel()} entries, the source has "
                             f"{nnz_written} non-zero words")
        return indices[:nnz_written].clone(), values[:nnz_written].clone()

    def get_profiling_stats(self) -> str:
        """The reference reports its native profiler; this converter keeps a
        call count only (torch_utils.py:118-125)."""
        return f"dense_to_sparse_32 calls: {self._calls}"
