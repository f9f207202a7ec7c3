"""CPU oracle for the LUT hot path -- TEST INFRASTRUCTURE ONLY.

Thin numpy/ctypes wrapper over ``liblut_oracle.so`` (built from
``lut_oracle.c`` by ``oracle/Makefile``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import
this package, and only as the checker; the product (``spiky_amd``) never does.

Every function restates the reference's single-threaded NO_CUDA path
(``spiky_cuda/misc/misc.h:119-129``); the per-function citations live in the
C source.  Arrays are numpy; outputs are accumulated into (as the reference
does), so pass zero-filled arrays for a plain result.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblut_oracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_int = ctypes.c_int


def build():
    """Compile liblut_oracle.so with the committed Makefile."""
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_decode_anchors_compact.argtypes = [_u32p, _i64, _i64, _i64, _i64p, _i32p, _i32p]
        L.oracle_decode_anchors_compact.restype = _i64
        L.oracle_check_detectors.argtypes = [_f32p, _i64, _i64, _i32p, _i64, _i64, _f32, _i32p, _vp, _vp]
        L.oracle_fill_outputs_fc.argtypes = [_vp, _vp, _vp, _i32p, _f32p, _i64, _i64, _i64, _i64, _i64, _int, _f64]
        L.oracle_convert_int_to_float.argtypes = [_f32p, _i64, _f64]
        L.oracle_propagate_fc.argtypes = [_f32p, _f32p, _i32p, _f32p, _i32p, _i32p, _f32p,
                                          _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _f64]
        L.oracle_gather_wgrad_fc.argtypes = [_f32p, _i32p, _f32p, _i64, _i64, _i64, _i64, _i64,
                                             _f32, _f32, _int, _f64]
        L.oracle_fill_outputs_sparse.argtypes = [_f32p, _i32p, _i64p, _i32p, _f32p, _i64, _i64, _i64,
                                                 _i64, _int, _f64]
        L.oracle_propagate_sparse.argtypes = [_f32p, _f32p, _i32p, _f32p, _i32p, _i32p, _i64p, _i32p,
                                              _f32p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                              _int, _f64]
        L.oracle_gather_wgrad_sparse.argtypes = [_f32p, _i32p, _i64p, _i32p, _f32p, _i64, _i64, _i64,
                                                 _i64, _f32, _f32, _int, _f64]
        L.oracle_check_pe.argtypes = [_f32p, _i64, _i64, _i64, _f32, _i32p, _vp, _vp]
        L.oracle_fill_outputs_seq.argtypes = [_f32p, _i32p, _vp, _f32p, _i64, _i64, _i64, _i64, _i64,
                                              _i64, _int, _f64]
        L.oracle_propagate_seq.argtypes = [_f32p, _f32p, _i32p, _f32p, _i32p, _vp, _vp, _vp, _i32p,
                                           _f32p, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                           _i64, _int, _f64, _vp, _vp]
        L.oracle_gather_wgrad_seq.argtypes = [_f32p, _i32p, _vp, _f32p, _i64, _i64, _i64, _i64, _i64,
                                              _i64, _i64, _f32, _f32, _int, _f64]
        L.oracle_fill_outputs_product.argtypes = [_f32p, _f32p, _vp, _i32p, _f32p, _i64, _i64, _i64, _i64,
                                                  _i64, _i64, _i64, _i64, _int, _f32, _int, _f64, _f32p]
        L.oracle_propagate_product.argtypes = [_f32p, _f32p, _vp, _i32p, _f32p, _f32p, _i64, _i64, _i64,
                                               _i64, _i64, _i64, _i64, _i64, _int, _f32, _f64, _int, _f64,
                                               _f32p, _f32p, _vp, _vp]
        L.oracle_fill_outputs_seq_sparse.argtypes = [_f32p, _i32p, _vp, _i64p, _i32p, _f32p, _i64, _i64,
                                                     _i64, _i64, _i64, _i64, _i64, _i64, _int, _f64]
        L.oracle_propagate_seq_sparse.argtypes = [_f32p, _f32p, _i32p, _f32p, _i32p, _vp, _vp, _vp, _i32p,
                                                  _i64p, _i32p, _f32p, _vp, _i64, _i64, _i64, _i64, _i64,
                                                  _i64, _i64, _i64, _i64, _int, _f64, _vp, _vp, _vp, _vp]
        L.oracle_gather_wgrad_seq_sparse.argtypes = [_f32p, _i32p, _vp, _i64p, _i32p, _f32p, _i64, _i64,
                                                     _i64, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _int,
                                                     _f64]
        L.oracle_fill_outputs_product_sparse.argtypes = [_f32p, _f32p, _vp, _i32p, _f32p, _i64p, _i32p,
                                                         _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                         _int, _f32, _int, _f64, _vp, _vp, _vp]
        L.oracle_propagate_product_sparse.argtypes = [_f32p, _f32p, _vp, _i32p, _f32p, _i64p, _i32p, _f32p,
                                                      _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int,
                                                      _f32, _f64, _int, _f64, _f32p, _f32p, _vp, _vp]
        L.oracle_propagate_product_sparse64.argtypes = [_f32p, _f32p, _vp, _i32p, _f32p, _i64p, _i32p,
                                                        _f32p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                        _i64, _int, _f32, _f64, _vp, _vp, _vp, _vp, _vp,
                                                        _vp, _vp, _vp]
        L.oracle_fill_outputs_product64.argtypes = [_f32p, _f32p, _vp, _i32p, _f32p, _i64, _i64, _i64,
                                                    _i64, _i64, _i64, _i64, _i64, _int, _f32, _vp, _vp]
        L.oracle_propagate_product64.argtypes = [_f32p, _f32p, _vp, _i32p, _f32p, _f32p, _i64, _i64,
                                                 _i64, _i64, _i64, _i64, _i64, _i64, _int, _f32, _f64,
                                                 _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- anchors
def decode_anchors_compact(encoded_pairs, n_detectors, max_pairs_per_detector, n_anchors,
                           in_offsets, in_ids):
    """Compact anchor decode; returns (anchors int32 [N_t*Nc*2], n_errors)."""
    out = np.zeros(n_detectors * n_anchors * 2, dtype=np.int32)
    err = lib().oracle_decode_anchors_compact(
        _c(encoded_pairs, np.int64).astype(np.uint32), n_detectors, max_pairs_per_detector,
        n_anchors, _c(in_offsets, np.int64), _c(in_ids, np.int32), out)
    return out, int(err)


# ---------------------------------------------------------------- FC path
def check_detectors(x, anchors, batch, n_inputs, n_detectors, n_anchors, cmp_eps=0.0, train=True):
    x = _c(x, np.float32)
    anchors = _c(anchors, np.int32)
    idx = np.zeros(batch * n_detectors, dtype=np.int32)
    md = np.zeros(batch * n_detectors, dtype=np.float32) if train else None
    mi = np.zeros(batch * n_detectors, dtype=np.int32) if train else None
    lib().oracle_check_detectors(x, batch, n_inputs, anchors, n_detectors, n_anchors,
                                 float(cmp_eps), idx, _ptr(md), _ptr(mi))
    return (idx, md, mi) if train else idx


def fill_outputs_fc(w, idx, batch, n_outputs, n_detectors, n_entries, dgs=32,
                    out=None, int_mode=False, int_rescaler=1.0, q8=None, scales=None):
    """Forward row gather-sum.  In int mode the result is the int32 accumulator
    (reinterpretation of `out`); call convert_int_to_float for the fp32 view."""
    if out is None:
        out = np.zeros(batch * n_outputs, dtype=np.float32)
    if q8 is not None:
        q8 = _c(q8, np.int8)
        scales = _c(scales, np.float32)
        w = None
    else:
        w = _c(w, np.float32)
    lib().oracle_fill_outputs_fc(_ptr(w), _ptr(q8), _ptr(scales), _c(idx, np.int32), out,
                                 batch, n_outputs, n_detectors, n_entries, dgs,
                                 int(int_mode), float(int_rescaler))
    return out


def convert_int_to_float(buf, int_rescaler):
    lib().oracle_convert_int_to_float(buf, buf.size, float(int_rescaler))
    return buf


def propagate_fc(w, g, idx, md, mi, anchors, batch, n_inputs, n_outputs, n_detectors,
                 n_anchors, n_entries, ogs=32, x_grad=None, int_mode=False, int_rescaler=1.0):
    if x_grad is None:
        x_grad = np.zeros(batch * n_inputs, dtype=np.float32)
    lib().oracle_propagate_fc(_c(w, np.float32), _c(g, np.float32), _c(idx, np.int32),
                              _c(md, np.float32), _c(mi, np.int32), _c(anchors, np.int32), x_grad,
                              batch, n_inputs, n_outputs, n_detectors, n_anchors, n_entries, ogs,
                              int(int_mode), float(int_rescaler))
    return x_grad


def gather_wgrad_fc(g, idx, target, batch, n_outputs, n_detectors, n_entries, ogs=32,
                    first_meta_lr=1.0, external_lr=-1.0, int_mode=False, int_rescaler=1.0):
    lib().oracle_gather_wgrad_fc(_c(g, np.float32), _c(idx, np.int32), target, batch, n_outputs,
                                 n_detectors, n_entries, ogs, float(first_meta_lr),
                                 float(external_lr), int(int_mode), float(int_rescaler))
    return target


# ---------------------------------------------------------------- sparse path
def fill_outputs_sparse(w, idx, syn_offsets, syn_targets, batch, n_outputs, n_detectors,
                        n_entries, out=None, int_mode=False, int_rescaler=1.0):
    if out is None:
        out = np.zeros(batch * n_outputs, dtype=np.float32)
    lib().oracle_fill_outputs_sparse(_c(w, np.float32), _c(idx, np.int32), _c(syn_offsets, np.int64),
                                     _c(syn_targets, np.int32), out, batch, n_outputs, n_detectors,
                                     n_entries, int(int_mode), float(int_rescaler))
    return out


def propagate_sparse(w, g, idx, md, mi, anchors, syn_offsets, syn_targets, batch, n_inputs,
                     n_outputs, n_detectors, n_anchors, n_entries, fgs, max_groups,
                     x_grad=None, int_mode=False, int_rescaler=1.0):
    if x_grad is None:
        x_grad = np.zeros(batch * n_inputs, dtype=np.float32)
    lib().oracle_propagate_sparse(_c(w, np.float32), _c(g, np.float32), _c(idx, np.int32),
                                  _c(md, np.float32), _c(mi, np.int32), _c(anchors, np.int32),
                                  _c(syn_offsets, np.int64), _c(syn_targets, np.int32), x_grad,
                                  batch, n_inputs, n_outputs, n_detectors, n_anchors, n_entries,
                                  fgs, max_groups, int(int_mode), float(int_rescaler))
    return x_grad


def gather_wgrad_sparse(g, idx, syn_offsets, syn_targets, target, batch, n_outputs, n_detectors,
                        n_entries, first_meta_lr=1.0, external_lr=-1.0, int_mode=False,
                        int_rescaler=1.0):
    lib().oracle_gather_wgrad_sparse(_c(g, np.float32), _c(idx, np.int32), _c(syn_offsets, np.int64),
                                     _c(syn_targets, np.int32), target, batch, n_outputs,
                                     n_detectors, n_entries, float(first_meta_lr),
                                     float(external_lr), int(int_mode), float(int_rescaler))
    return target


# ---------------------------------------------------------------- sequence-concat path
def check_pe(pe, seq_len, n_detectors, positional_dim, cmp_eps=0.0, train=True):
    """Positional lookup indices [(S-1)][T] (and min margins in train mode)."""
    n = (seq_len - 1) * n_detectors
    pidx = np.zeros(n, dtype=np.int32)
    pmd = np.zeros(n, dtype=np.float32) if train else None
    pmi = np.zeros(n, dtype=np.int32) if train else None
    lib().oracle_check_pe(_c(pe, np.float32), seq_len, n_detectors, positional_dim, float(cmp_eps),
                          pidx, _ptr(pmd), _ptr(pmi))
    return (pidx, pmd, pmi) if train else pidx


def fill_outputs_seq(w, idx, pidx, batch, n_outputs, n_detectors, seq_len, n_anchors,
                     positional_dim, out=None, int_mode=False, int_rescaler=1.0):
    if out is None:
        out = np.zeros(batch * seq_len * n_outputs, dtype=np.float32)
    pidx = None if pidx is None else _c(pidx, np.int32)
    lib().oracle_fill_outputs_seq(_c(w, np.float32), _c(idx, np.int32), _ptr(pidx), out, batch,
                                  n_outputs, n_detectors, seq_len, n_anchors, positional_dim,
                                  int(int_mode), float(int_rescaler))
    return out


def propagate_seq(w, g, idx, md, mi, pidx, pmd, pmi, anchors, batch, n_inputs, n_outputs,
                  n_detectors, seq_len, n_anchors, positional_dim, ogs=32, x_grad=None,
                  pe_grad=None, int_mode=False, int_rescaler=1.0, acc64=False):
    """Returns (x_grad [B*S*I], pe_grad [(S-1)*T*Npe] or None).  With acc64
    (fp32 summation) the same terms are summed in fp64 and returned as float64
    arrays: the reference's sums without the fp32 rounding of each partial."""
    if x_grad is None:
        x_grad = np.zeros(batch * seq_len * n_inputs, dtype=np.float32)
    if pe_grad is None and positional_dim > 0:
        pe_grad = np.zeros((seq_len - 1) * n_detectors * positional_dim, dtype=np.float32)
    xg64 = pg64 = None
    if acc64 and not int_mode:
        xg64 = np.zeros(batch * seq_len * n_inputs, dtype=np.float64)
        if positional_dim > 0:
            pg64 = np.zeros((seq_len - 1) * n_detectors * positional_dim, dtype=np.float64)
    pidx, pmd, pmi = (None if a is None else _c(a, dt) for a, dt in
                      ((pidx, np.int32), (pmd, np.float32), (pmi, np.int32)))
    lib().oracle_propagate_seq(_c(w, np.float32), _c(g, np.float32), _c(idx, np.int32),
                               _c(md, np.float32), _c(mi, np.int32), _ptr(pidx), _ptr(pmd),
                               _ptr(pmi), _c(anchors, np.int32), x_grad, _ptr(pe_grad), batch,
                               n_inputs, n_outputs, n_detectors, seq_len, n_anchors,
                               positional_dim, ogs, int(int_mode), float(int_rescaler),
                               _ptr(xg64), _ptr(pg64))
    if xg64 is not None:
        return xg64, pg64
    return x_grad, pe_grad


def gather_wgrad_seq(g, idx, pidx, target, batch, n_outputs, n_detectors, seq_len, n_anchors,
                     positional_dim, ogs=32, first_meta_lr=1.0, external_lr=-1.0,
                     int_mode=False, int_rescaler=1.0):
    pidx = None if pidx is None else _c(pidx, np.int32)
    lib().oracle_gather_wgrad_seq(_c(g, np.float32), _c(idx, np.int32), _ptr(pidx), target, batch,
                                  n_outputs, n_detectors, seq_len, n_anchors, positional_dim, ogs,
                                  float(first_meta_lr), float(external_lr), int(int_mode),
                                  float(int_rescaler))
    return target


def dense_to_sparse_32(source):
    """Non-zero 32-bit words of a 1-D array: (int64 indices ascending, values
    of the same dtype).  A word counts as non-zero when its bit pattern is
    non-zero, as in the reference's int4 compare (densify_logic,
    spiky_cuda/torch_utils/torch_utils_kernels_logic.proto:20-35), so a float
    -0.0 is kept.  The reference orders its output only within a block; this
    restatement (and the HIP path) orders it by index."""
    src = np.ascontiguousarray(source)
    if src.dtype.itemsize != 4:
        raise ValueError("source must be 32-bit")
    bits = src.view(np.uint32)
    idx = np.flatnonzero(bits).astype(np.int64)
    return idx, src[idx].copy()


def fill_outputs_product(x1, x2, pe, anchors, w, batch, seq_len, n1, n2, pd, n_detectors, n_anchors,
                         n_outputs, sliced=False, cmp_eps=0.0, int_mode=False, int_rescaler=1.0,
                         out=None):
    """Product-mode forward (fill_outputs_product_cpu_logic, proto:2148-2264):
    out [B*S*O] accumulated into; x1 [B*S*n1], x2 [B*S*n2], pe [(S-1)*T*pd] or
    None, anchors int32 pairs [T*Nc*2] (-1 = unused) over the virtual row."""
    if out is None:
        out = np.zeros(batch * seq_len * n_outputs, dtype=np.float32)
    pe = None if pe is None or pd == 0 else _c(pe, np.float32)
    lib().oracle_fill_outputs_product(_c(x1, np.float32), _c(x2, np.float32), _ptr(pe),
                                      _c(anchors, np.int32), _c(w, np.float32), batch, seq_len, n1,
                                      n2, pd, n_detectors, n_anchors, n_outputs, int(sliced),
                                      float(cmp_eps), int(int_mode), float(int_rescaler), out)
    return out


def propagate_product(x1, x2, pe, anchors, w, g, batch, seq_len, n1, n2, pd, n_detectors, n_anchors,
                      n_outputs, sliced=False, cmp_eps=0.0, lr=1.0, int_mode=False,
                      int_rescaler=1.0, x_grad=None, pe_grad=None, w_grad=None, same_x=True):
    """Product-mode backward (propagate_backward_product_cpu_logic,
    proto:2396-2628).  With same_x (the layer's call: x1 is x2) both roles
    accumulate into one x_grad [B*S*n1]; returns (x_grad, pe_grad, w_grad)
    (x2_grad appended when not same_x).  w_grad None skips the weight
    gradient (Internal policy)."""
    if x_grad is None:
        x_grad = np.zeros(batch * seq_len * n1, dtype=np.float32)
    x2_grad = x_grad if same_x else np.zeros(batch * seq_len * n2, dtype=np.float32)
    if pe_grad is None and pd > 0:
        pe_grad = np.zeros((seq_len - 1) * n_detectors * pd, dtype=np.float32)
    pe = None if pe is None or pd == 0 else _c(pe, np.float32)
    lib().oracle_propagate_product(_c(x1, np.float32), _c(x2, np.float32), _ptr(pe),
                                   _c(anchors, np.int32), _c(w, np.float32), _c(g, np.float32), batch,
                                   seq_len, n1, n2, pd, n_detectors, n_anchors, n_outputs, int(sliced),
                                   float(cmp_eps), float(lr), int(int_mode), float(int_rescaler),
                                   x_grad, x2_grad, _ptr(pe_grad), _ptr(w_grad))
    if same_x:
        return x_grad, pe_grad, w_grad
    return x_grad, pe_grad, w_grad, x2_grad


def fill_outputs_product64(x1, x2, pe, anchors, w, batch, seq_len, n1, n2, pd, n_detectors, n_anchors,
                           n_outputs, sliced=False, cmp_eps=0.0):
    """fp64 mode of fill_outputs_product: (sum, abs) of the reference's terms
    per output, in float64.  Any fp32 summation order of n terms lies within
    n * 2^-24 * abs of sum (the tolerance of an order-free GPU sum)."""
    m = batch * seq_len * n_outputs
    tot, mag = np.zeros(m), np.zeros(m)
    pe = None if pe is None or pd == 0 else _c(pe, np.float32)
    lib().oracle_fill_outputs_product64(_c(x1, np.float32), _c(x2, np.float32), _ptr(pe),
                                        _c(anchors, np.int32), _c(w, np.float32), batch, seq_len, n1,
                                        n2, pd, n_detectors, n_anchors, n_outputs, int(sliced),
                                        float(cmp_eps), _ptr(tot), _ptr(mag))
    return tot, mag


def propagate_product64(x1, x2, pe, anchors, w, g, batch, seq_len, n1, n2, pd, n_detectors, n_anchors,
                        n_outputs, sliced=False, cmp_eps=0.0, lr=1.0, weights=True):
    """fp64 mode of propagate_product with x1 is x2 (the layer's call):
    returns {"x", "pe", "w"} -> (sum, abs) of the terms ((float)du pushes,
    (float)(g*lr) gradient terms); "w" is None when weights is False."""
    nx = batch * seq_len * n1
    x_s, x_a = np.zeros(nx), np.zeros(nx)
    npe = (seq_len - 1) * n_detectors * pd
    pe_s, pe_a = (np.zeros(npe), np.zeros(npe)) if pd > 0 else (None, None)
    nw = (n_detectors << n_anchors) * n_outputs
    w_s, w_a = (np.zeros(nw), np.zeros(nw)) if weights else (None, None)
    pe = None if pe is None or pd == 0 else _c(pe, np.float32)
    lib().oracle_propagate_product64(_c(x1, np.float32), _c(x2, np.float32), _ptr(pe),
                                     _c(anchors, np.int32), _c(w, np.float32), _c(g, np.float32), batch,
                                     seq_len, n1, n2, pd, n_detectors, n_anchors, n_outputs, int(sliced),
                                     float(cmp_eps), float(lr), _ptr(x_s), _ptr(x_a), _ptr(x_s),
                                     _ptr(x_a), _ptr(pe_s), _ptr(pe_a), _ptr(w_s), _ptr(w_a))
    return {"x": (x_s, x_a), "pe": (pe_s, pe_a) if pd > 0 else None,
            "w": (w_s, w_a) if weights else None}


# ---------------------------------------------------------------- sequence-concat, sparse
def fill_outputs_seq_sparse(w, idx, pidx, syn_offsets, syn_targets, batch, seq_len, n_outputs, n_detectors,
                            n_anchors, positional_dim, fgs, max_groups, int_mode=False, int_rescaler=1.0,
                            out=None):
    """Sequence-concat forward over sparse connectivity (proto:1906-2015):
    out [B*S*O] accumulated into; idx [B*S*T]; pidx [(S-1)*T] or None."""
    if out is None:
        out = np.zeros(batch * seq_len * n_outputs, dtype=np.float32)
    pidx = None if pidx is None or positional_dim == 0 else _c(pidx, np.int32)
    lib().oracle_fill_outputs_seq_sparse(_c(w, np.float32), _c(idx, np.int32), _ptr(pidx),
                                         _c(syn_offsets, np.int64), _c(syn_targets, np.int32), out, batch,
                                         seq_len, n_outputs, n_detectors, n_anchors, positional_dim, fgs,
                                         max_groups, int(int_mode), float(int_rescaler))
    return out


def propagate_seq_sparse(w, g, idx, md, mi, pidx, pmd, pmi, anchors, syn_offsets, syn_targets, batch,
                         n_inputs, n_outputs, n_detectors, seq_len, n_anchors, positional_dim, fgs,
                         max_groups, int_mode=False, int_rescaler=1.0, bounds=False):
    """Sequence-concat backward into x / pe over sparse connectivity
    (proto:3371-3627).  Returns (x_grad, pe_grad) and, with bounds, also
    ((x_sum, x_abs), (pe_sum, pe_abs)): the pushes in fp64 and their magnitudes."""
    x_grad = np.zeros(batch * seq_len * n_inputs, dtype=np.float32)
    npe = (seq_len - 1) * n_detectors * positional_dim
    pe_grad = np.zeros(npe, dtype=np.float32) if positional_dim > 0 else None
    xs = xa = ps = pa = None
    if bounds:
        xs, xa = np.zeros(x_grad.size), np.zeros(x_grad.size)
        if positional_dim > 0:
            ps, pa = np.zeros(npe), np.zeros(npe)
    pd = positional_dim > 0
    lib().oracle_propagate_seq_sparse(
        _c(w, np.float32), _c(g, np.float32), _c(idx, np.int32), _c(md, np.float32), _c(mi, np.int32),
        _ptr(_c(pidx, np.int32) if pd else None), _ptr(_c(pmd, np.float32) if pd else None),
        _ptr(_c(pmi, np.int32) if pd else None), _c(anchors, np.int32), _c(syn_offsets, np.int64),
        _c(syn_targets, np.int32), x_grad, _ptr(pe_grad), batch, n_inputs, n_outputs, n_detectors,
        seq_len, n_anchors, positional_dim, fgs, max_groups, int(int_mode), float(int_rescaler),
        _ptr(xs), _ptr(xa), _ptr(ps), _ptr(pa))
    if bounds:
        return x_grad, pe_grad, (xs, xa), ((ps, pa) if pd else None)
    return x_grad, pe_grad


def gather_wgrad_seq_sparse(g, idx, pidx, syn_offsets, syn_targets, batch, seq_len, n_outputs,
                            n_detectors, n_anchors, positional_dim, fgs, max_groups, lr=1.0,
                            external_lr=-1.0, int_mode=False, int_rescaler=1.0, target=None):
    """Sequence-concat weight gradient over sparse connectivity
    (proto:3837-3942) into target [n_synapses]."""
    if target is None:
        target = np.zeros(int(np.asarray(syn_offsets)[-1]), dtype=np.float32)
    pidx = None if pidx is None or positional_dim == 0 else _c(pidx, np.int32)
    lib().oracle_gather_wgrad_seq_sparse(_c(g, np.float32), _c(idx, np.int32), _ptr(pidx),
                                         _c(syn_offsets, np.int64), _c(syn_targets, np.int32), target,
                                         batch, seq_len, n_outputs, n_detectors, n_anchors,
                                         positional_dim, fgs, max_groups, float(lr), float(external_lr),
                                         int(int_mode), float(int_rescaler))
    return target


# ---------------------------------------------------------------- product mode, sparse
def fill_outputs_product_sparse(x1, x2, pe, anchors, w, syn_offsets, syn_targets, batch, seq_len, n1, n2,
                                pd, n_detectors, n_anchors, n_outputs, sliced=False, cmp_eps=0.0,
                                int_mode=False, int_rescaler=1.0, bounds=False):
    """Product-mode forward over sparse connectivity (w per synapse).  Returns
    out [B*S*O] (fp32 / int32 payloads), or with bounds the fp64 (sum, abs)
    of the terms."""
    m = batch * seq_len * n_outputs
    out = np.zeros(m, dtype=np.float32)
    tot = mag = None
    if bounds:
        tot, mag = np.zeros(m), np.zeros(m)
    pe = None if pe is None or pd == 0 else _c(pe, np.float32)
    lib().oracle_fill_outputs_product_sparse(
        _c(x1, np.float32), _c(x2, np.float32), _ptr(pe), _c(anchors, np.int32), _c(w, np.float32),
        _c(syn_offsets, np.int64), _c(syn_targets, np.int32), batch, seq_len, n1, n2, pd, n_detectors,
        n_anchors, n_outputs, int(sliced), float(cmp_eps), int(int_mode), float(int_rescaler),
        None if bounds else _ptr(out), _ptr(tot), _ptr(mag))
    return (tot, mag) if bounds else out


def propagate_product_sparse(x1, x2, pe, anchors, w, syn_offsets, syn_targets, g, batch, seq_len, n1, n2,
                             pd, n_detectors, n_anchors, n_outputs, sliced=False, cmp_eps=0.0, lr=1.0,
                             int_mode=False, int_rescaler=1.0, weights=True, bounds=False):
    """Product-mode backward over sparse connectivity with x1 is x2.  Returns
    (x_grad, pe_grad, w_grad [n_synapses] or None) or, with bounds,
    {"x", "pe", "w"} -> fp64 (sum, abs) of the terms."""
    nx = batch * seq_len * n1
    npe = (seq_len - 1) * n_detectors * pd
    nsyn = int(np.asarray(syn_offsets)[-1])
    pe = None if pe is None or pd == 0 else _c(pe, np.float32)
    common = (_c(x1, np.float32), _c(x2, np.float32), _ptr(pe), _c(anchors, np.int32), _c(w, np.float32),
              _c(syn_offsets, np.int64), _c(syn_targets, np.int32), _c(g, np.float32), batch, seq_len, n1,
              n2, pd, n_detectors, n_anchors, n_outputs, int(sliced), float(cmp_eps), float(lr))
    if bounds:
        xs, xa = np.zeros(nx), np.zeros(nx)
        ps, pa = (np.zeros(npe), np.zeros(npe)) if pd > 0 else (None, None)
        ws, wa = (np.zeros(nsyn), np.zeros(nsyn)) if weights else (None, None)
        lib().oracle_propagate_product_sparse64(*common, _ptr(xs), _ptr(xa), _ptr(xs), _ptr(xa), _ptr(ps),
                                                _ptr(pa), _ptr(ws), _ptr(wa))
        return {"x": (xs, xa), "pe": (ps, pa) if pd > 0 else None, "w": (ws, wa) if weights else None}
    x_grad = np.zeros(nx, dtype=np.float32)
    pe_grad = np.zeros(npe, dtype=np.float32) if pd > 0 else None
    w_grad = np.zeros(nsyn, dtype=np.float32) if weights else None
    lib().oracle_propagate_product_sparse(*common, int(int_mode), float(int_rescaler), x_grad, x_grad,
                                          _ptr(pe_grad), _ptr(w_grad))
    return x_grad, pe_grad, w_grad
