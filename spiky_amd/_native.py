"""Loader of libspiky_lut.so, the HIP kernels behind the C ABI in include/spiky_lut.h.

The library is built in-tree (``python -m spiky_amd.build``).  There is no
fallback: if the library is missing or fails to load, every device entry point
raises, so a GPU run can never silently compute somewhere else.
"""
import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libspiky_lut.so")

SPIKY_OK = 0
SPIKY_VALUE_ERROR = 1
SPIKY_RUNTIME_ERROR = 2

_lock = threading.Lock()
_lib = None

_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_vp = ctypes.c_void_p
_pp = ctypes.POINTER(ctypes.c_void_p)

_SIGNATURES = {
    "spiky_lut_last_error": ([], ctypes.c_char_p),
    "spiky_lut_version": ([], ctypes.c_char_p),
    "spiky_lut_create": ([_u32, _u32, _u32, _u32, _u32, _u32, _u64, _u32, _u32, _i32, _f64, _pp], _i32),
    "spiky_lut_destroy": ([_vp], None),
    "spiky_lut_set_ordered_sums": ([_vp, _i32], _i32),
    "spiky_lut_register_synapse_meta": ([_vp, _f32, _f32, _f32, _f32, _f32, ctypes.POINTER(_u32)], _i32),
    "spiky_lut_initialize_neurons": ([_vp, _i32], _i32),
    "spiky_lut_n_lookup_neurons": ([_vp], _u64),
    "spiky_lut_weights_dimension": ([_vp], _u64),
    "spiky_lut_max_forward_groups_per_neuron": ([_vp], _u32),
    "spiky_lut_n_synapses": ([_vp], _u64),
    "spiky_lut_forward_step": ([_vp, _vp, _u32, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp], _i32),
    "spiky_lut_forward_step_noalloc": ([_vp, _vp, _u32, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp], _i32),
    "spiky_lut_forward_step_i8": ([_vp, _vp, _vp, _u32, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp], _i32),
    "spiky_lut_backward_backprop": ([_vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _f64, _vp, _i32, _vp], _i32),
    "spiky_lut_set_sparse_connectivity": ([_vp, _vp, _vp, _u64], _i32),
    "spiky_lut_decode_anchors_compact": ([_vp, _u32, _u32, _u32, _vp, _vp, _vp], _i32),
    "spiky_lut_profiling_stats": ([_vp, ctypes.c_char_p, _u64], _i32),
    "spiky_lut_reset_profiler": ([_vp], None),
    "spiky_lut_set_kernel_timing": ([_vp, _i32], _i32),
    "spiky_lut_kernel_times": ([_vp, ctypes.c_char_p, _u64, _i32], _i32),
    "spiky_lut_scratch_plan": ([_vp, _i32, _u32, _u32, _u32, _u32, _i32, _u64, _vp], _i32),
    "spiky_grow_cuboid": ([_u32, _vp, _vp, _u32, _vp, _vp, _vp, _f32, _u64, _u32, _vp, _vp, _u64,
                           ctypes.POINTER(_u64)], _i32),
    "spiky_densify32_workspace_bytes": ([_u64], _u64),
    "spiky_count_nonzero32": ([_vp, _u64, _vp, _u64, _vp, _vp], _i32),
    "spiky_dense_to_sparse32": ([_vp, _u64, _vp, _vp, _u64, _vp, _u64, _vp, _i32, _i32, _vp], _i32),
}

# Sequence-mode entry points are bound when the library exports them.
_OPTIONAL_SIGNATURES = {
    "spiky_lut_forward_step_concat": (
        [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "spiky_lut_backward_backprop_concat": (
        [_vp, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _f64, _vp, _vp, _vp, _vp, _vp, _i32, _vp], _i32),
    "spiky_lut_forward_step_product": (
        [_vp, _vp, _u32, _u32, _vp, _vp, _vp, _vp, _u32, _u32, _i32, _f32, _vp, _vp], _i32),
    "spiky_lut_backward_backprop_product": (
        [_vp, _vp, _u32, _u32, _vp, _vp, _vp, _vp, _vp, _vp, _f64, _u32, _u32, _i32, _f32, _vp, _vp,
         _vp, _vp], _i32),
}


def exported_symbols():
    """Names of every C-ABI entry point this module binds."""
    return list(_SIGNATURES) + list(_OPTIONAL_SIGNATURES)


def lib():
    """Load (once) and return the ctypes handle; raises if the library is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"spiky_amd native library not found at {LIB_PATH}; build it with "
                "`python -m spiky_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        for name, (args, res) in _OPTIONAL_SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is not None:
                fn.argtypes = args
                fn.restype = res
        _lib = L
    return _lib


def check(status):
    """Map a C-ABI status to the reference's Python exception types."""
    if status == SPIKY_OK:
        return
    msg = lib().spiky_lut_last_error().decode("utf-8", "replace")
    if status == SPIKY_VALUE_ERROR:
        raise ValueError(msg)
    raise RuntimeError(msg)
