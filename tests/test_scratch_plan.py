"""Scratch layouts of every entry point against the buffer it requests, on the
host (no GPU): spiky_lut_scratch_plan reports the bytes an entry point grows
its scratch buffer to and checks each launcher's layout against its region of
a buffer of a given capacity, in the same code the entry points run before
launching anything.  For BASELINE configs 1-5, the product-mode attention
layer and the shapes the GPU tests use:

  * the requested buffer holds every launcher's layout (for the fully
    connected backward: the propagate's region, then the weight gradient's);
  * one byte less is refused with a message naming the launcher and the bytes
    its layout needs (the entry points refuse it the same way, before any
    launch, instead of writing past the buffer);
  * the sizes the documentation quotes for config 3 hold.
"""
import ctypes

import pytest

from spiky_amd import LUTDataManagerF, LUTDataManagerI, _native

OPS = dict(FORWARD=0, FORWARD_I8=1, BACKWARD=2, BACKWARD_NO_WGRAD=3, FORWARD_CONCAT=4,
           BACKWARD_CONCAT=5, FORWARD_PRODUCT=6, BACKWARD_PRODUCT=7)
NO_LIMIT = (1 << 64) - 1


def manager(I, O, T, Nc, S=1, Npe=0, int_rescaler=None, fc=True):
    if int_rescaler is None:
        dm = LUTDataManagerF(I, O, T, Nc, S, Npe, 0, 32, 32)
    else:
        dm = LUTDataManagerI(I, O, T, Nc, S, Npe, 0, 32, 32, int_rescaler)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(fc)
    return dm


def plan(dm, op, B, S=0, n1=0, n2=0, sliced=0, capacity=NO_LIMIT):
    need = ctypes.c_uint64(0)
    rc = _native.lib().spiky_lut_scratch_plan(dm._h, OPS[op], B, S, n1, n2, sliced, capacity,
                                              ctypes.byref(need))
    return rc, need.value


def walk(dm, op, B, **kw):
    """The requested bytes fit every launcher's layout; one byte less does not."""
    rc, need = plan(dm, op, B, **kw)
    assert rc == _native.SPIKY_OK, _native.lib().spiky_lut_last_error()
    rc2, need2 = plan(dm, op, B, capacity=need, **kw)
    assert (rc2, need2) == (_native.SPIKY_OK, need), _native.lib().spiky_lut_last_error()
    if need:
        rc3, _ = plan(dm, op, B, capacity=need - 1, **kw)
        assert rc3 == _native.SPIKY_VALUE_ERROR
        msg = _native.lib().spiky_lut_last_error().decode()
        assert "scratch layout needs" in msg and "given" in msg, msg
    return need


CASES = [
    # BASELINE config 1 (B 64: the small-batch kernels, only the weight gradient's buckets)
    ("config1", dict(I=784, O=10, T=256, Nc=6), 64, ["FORWARD", "BACKWARD", "BACKWARD_NO_WGRAD"]),
    # config 3 and its int32-summation form
    ("config3", dict(I=4096, O=1024, T=8192, Nc=8), 1024, ["FORWARD", "BACKWARD", "BACKWARD_NO_WGRAD"]),
    ("config3_int32", dict(I=4096, O=1024, T=8192, Nc=8, int_rescaler=0.001), 1024,
     ["FORWARD", "BACKWARD", "BACKWARD_NO_WGRAD"]),
    # config 4: int8 tables, int32 sums, B 4096
    ("config4", dict(I=4096, O=1024, T=8192, Nc=8, int_rescaler=0.001), 4096, ["FORWARD_I8", "FORWARD"]),
    # config 5: attention layers (sequence concat) and the FC layers over B*S rows
    ("config5_attention", dict(I=256, O=256, T=64, Nc=6, S=256, Npe=4), 32,
     ["FORWARD_CONCAT", "BACKWARD_CONCAT"]),
    ("config5_attention_int32", dict(I=256, O=256, T=64, Nc=6, S=256, Npe=4, int_rescaler=0.25), 32,
     ["FORWARD_CONCAT", "BACKWARD_CONCAT"]),
    ("config5_ffn", dict(I=256, O=256, T=16, Nc=8), 8192, ["FORWARD", "BACKWARD"]),
    # shapes of the GPU tests: odd sizes, the pair-parallel sequence pass, the
    # allocation-free forward
    ("ragged_fc", dict(I=96, O=100, T=37, Nc=5), 515, ["FORWARD", "BACKWARD"]),
    ("seq_pairs", dict(I=24, O=100, T=3, Nc=3, S=40, Npe=3), 2, ["FORWARD_CONCAT", "BACKWARD_CONCAT"]),
    ("seq_one_bucket", dict(I=16, O=96, T=2, Nc=3, S=64, Npe=2), 160, ["FORWARD_CONCAT", "BACKWARD_CONCAT"]),
    ("noalloc", dict(I=256, O=256, T=512, Nc=8), 1024, ["FORWARD"]),
]


@pytest.mark.parametrize("name,shape,B,ops", CASES, ids=[c[0] for c in CASES])
def test_layouts_fit_requested_buffers(name, shape, B, ops):
    dm = manager(**shape)
    for op in ops:
        walk(dm, op, B)


def test_product_mode_layouts():
    # the product-mode attention layer of bench.py --product (B 32, S 256,
    # n 256, 64 tables of 6 anchors, pd 4, O 256): the manager takes the
    # virtual row [x_i | x_j | pe] as its inputs
    dm = manager(2 * 256 + 4, 256, 64, 6, S=1, Npe=4)
    for op in ("FORWARD_PRODUCT", "BACKWARD_PRODUCT"):
        need = walk(dm, op, 32, S=256, n1=256, n2=256)
        # Cnt [B*S][T*E] fp32 at least (and P in fp64 in the backward)
        assert need >= 32 * 256 * 64 * 64 * 4
    walk(dm, "FORWARD_PRODUCT", 3, S=9, n1=256, n2=256, sliced=1)


def test_sparse_layouts():
    # sparse connectivity: only the weight gradient's buckets use scratch
    import numpy as np
    dm = manager(20, 12, 4, 3, fc=False)
    E = 8
    n_lookup = 4 * E
    offs = np.arange(n_lookup + 1, dtype=np.int64) * 3
    tg = (np.arange(n_lookup * 3) % 12).astype(np.int32)
    _native.check(_native.lib().spiky_lut_set_sparse_connectivity(
        dm._h, offs.ctypes.data_as(ctypes.c_void_p), tg.ctypes.data_as(ctypes.c_void_p), tg.size))
    assert walk(dm, "FORWARD", 100) == 0
    assert walk(dm, "BACKWARD", 100) > 0
    assert walk(dm, "BACKWARD_NO_WGRAD", 100) == 0


@pytest.mark.parametrize("Nc,key_bytes", [(3, 1), (9, 2)])
def test_uniform_sparse_forward_layout(Nc, key_bytes):
    # every lookup neuron of a detector sharing its target list: from a batch of
    # 48 the forward lays the lookup indices out table-major, one byte a key for
    # up to 256 rows and two beyond
    import numpy as np
    T, O = 5, 12
    dm = manager(20, O, T, Nc, fc=False)
    E = 1 << Nc
    row = [np.array([(3 * t + k) % O for k in range(3 + t % 2)], np.int32) for t in range(T)]
    tg = np.concatenate([np.tile(row[t], E) for t in range(T)]).astype(np.int32)
    lens = np.repeat([len(r) for r in row], E)
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    _native.check(_native.lib().spiky_lut_set_sparse_connectivity(
        dm._h, offs.ctypes.data_as(ctypes.c_void_p), tg.ctypes.data_as(ctypes.c_void_p), tg.size))
    assert walk(dm, "FORWARD", 47) == 0
    assert walk(dm, "FORWARD", 48) == T * 48 * key_bytes
    assert walk(dm, "FORWARD", 1000) == T * 1000 * key_bytes


def test_config3_sizes():
    """Config 3's scratch: the forward's transposed u8 indices [T][B] and one
    fp32 partial [B][O] per unit of eight folded 32-table blocks; the
    backward's u32 keys and du values [T][B], du [B][T], then the weight
    gradient's bucket offsets [T][E+1], sorted samples [T][B] and commit
    values [B][O] (256-byte aligned regions)."""
    B, I, T, Nc, O = 1024, 4096, 8192, 8, 1024
    E = 1 << Nc
    dm = manager(I, O, T, Nc)
    fwd = walk(dm, "FORWARD", B)
    assert fwd == T * B + (T // 32 // 8) * B * O * 4
    bwd = walk(dm, "BACKWARD", B)
    prop = 3 * T * B * 4
    align = lambda n: (n + 255) // 256 * 256
    assert bwd == prop + align(T * (E + 1) * 4) + align(T * B * 4) + B * O * 4
    assert fwd < 0.15e9 and bwd < 0.16e9
    # ordered sums keep one partial per 32-table block
    _native.check(_native.lib().spiky_lut_set_ordered_sums(dm._h, 1))
    assert walk(dm, "FORWARD", B) == T * B + (T // 32) * B * O * 4


def test_allocation_free_limit():
    # the allocation-free forward's static array holds 64 MiB: the GPU test's
    # refused shape (B 8192) needs more, its accepted ones (1024, 300) less
    dm = manager(256, 256, 512, 8)
    assert walk(dm, "FORWARD", 1024) <= 64 << 20
    assert walk(dm, "FORWARD", 8192) > 64 << 20


def test_plan_validation():
    dm = manager(16, 8, 4, 3)
    lib = _native.lib()
    need = ctypes.c_uint64(0)
    assert lib.spiky_lut_scratch_plan(dm._h, 99, 4, 0, 0, 0, 0, NO_LIMIT, ctypes.byref(need)) == \
        _native.SPIKY_VALUE_ERROR
    assert b"unknown operation" in lib.spiky_lut_last_error()
    assert lib.spiky_lut_scratch_plan(dm._h, 0, 0, 0, 0, 0, 0, NO_LIMIT, ctypes.byref(need)) == \
        _native.SPIKY_VALUE_ERROR
    assert lib.spiky_lut_scratch_plan(dm._h, OPS["FORWARD_CONCAT"], 4, 0, 0, 0, 0, NO_LIMIT,
                                      ctypes.byref(need)) == _native.SPIKY_VALUE_ERROR
    assert b"sequence_length > 1" in lib.spiky_lut_last_error()
