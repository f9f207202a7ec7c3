"""spiky_lut_forward_step_noalloc (the allocation-free forward) against
spiky_lut_forward_step, through the C ABI: two calls in a row on one
manager, the second with a smaller batch, both on the table-major path whose
scratch is the library's static device array; then a shape beyond that
array's size is refused before any launch.  Indices, margins and outputs must
be bit-identical to the allocating entry point's (fp32 and int32 summation)."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("int_mode", [False, True])
def test_forward_noalloc_matches_forward(cuda_device, int_mode):
    from spiky_amd import LUTDataManagerF, LUTDataManagerI, _native
    dev = cuda_device
    L = _native.lib()
    I, T, Nc, O = 256, 512, 8, 256
    E = 1 << Nc
    if int_mode:
        dm = LUTDataManagerI(I, O, T, Nc, 1, 0, 0, 32, 32, 0.001)
    else:
        dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, 32, 32)
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    g = torch.Generator().manual_seed(23)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten().to(dev)
    W = (torch.randn(T * E * O, generator=g) * 0.01).to(dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for B in (1024, 300):   # the second call smaller: stale scratch contents must not leak
        print(f"[noalloc] int={int_mode} B={B}", flush=True)
        x = torch.randn(B * I, generator=g).to(dev)
        outs = []
        for fn in (L.spiky_lut_forward_step, L.spiky_lut_forward_step_noalloc):
            out = torch.zeros(B * O, device=dev)
            idx = torch.full((B * T,), -7, dtype=torch.int32, device=dev)
            md = torch.full((B * T,), 9.0, device=dev)
            mi = torch.full((B * T,), -7, dtype=torch.int32, device=dev)
            _native.check(fn(dm._h, _p(W), B, _p(x), _p(anchors), _p(out), _p(idx), ctypes.c_float(0.0),
                             _p(md), _p(mi), stream))
            torch.cuda.synchronize()
            outs.append((out.cpu(), idx.cpu(), md.cpu(), mi.cpu()))
        for a, b in zip(*outs):
            assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a,
                               b.view(torch.int32) if b.dtype == torch.float32 else b)
    # a batch whose block partials exceed the static scratch is refused, nothing launched
    B = 8192
    need = T // 32 * B * O * 4
    assert need > (64 << 20)
    x = torch.zeros(B * I, device=dev)
    out = torch.zeros(B * O, device=dev)
    idx = torch.zeros(B * T, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="bytes of scratch"):
        _native.check(L.spiky_lut_forward_step_noalloc(dm._h, _p(W), B, _p(x), _p(anchors), _p(out), _p(idx),
                                                       ctypes.c_float(0.0), None, None, stream))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0


def test_forward_noalloc_two_streams_back_to_back(cuda_device):
    """Two allocation-free calls issued back to back on two streams (one
    manager each, different batches, no host synchronisation between them)
    share the device's static array; the second call waits for the first's
    kernels, so both equal the allocating entry point's results bit for bit."""
    from spiky_amd import LUTDataManagerF, _native
    dev = cuda_device
    L = _native.lib()
    I, T, Nc, O = 256, 512, 8, 256
    E = 1 << Nc
    g = torch.Generator().manual_seed(29)
    anchors = torch.stack([torch.randperm(I, generator=g)[:2] for _ in range(T * Nc)]).to(torch.int32).flatten().to(dev)
    W = (torch.randn(T * E * O, generator=g) * 0.01).to(dev)
    dms, cases = [], []
    for B in (1024, 640):
        dm = LUTDataManagerF(I, O, T, Nc, 1, 0, 0, 32, 32)
        dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
        dm.initialize_neurons(True)
        dm.to_device(0)
        dms.append(dm)
        x = torch.randn(B * I, generator=g).to(dev)
        cases.append((B, x))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    got = []
    for dm, (B, x), s in zip(dms, cases, streams):
        out = torch.zeros(B * O, device=dev)
        idx = torch.empty(B * T, dtype=torch.int32, device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        print(f"[noalloc two streams] B={B}", flush=True)
        _native.check(L.spiky_lut_forward_step_noalloc(dm._h, _p(W), B, _p(x), _p(anchors), _p(out), _p(idx),
                                                       ctypes.c_float(0.0), None, None,
                                                       ctypes.c_void_p(s.cuda_stream)))
        got.append((out, idx))
    torch.cuda.synchronize()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for dm, (B, x), (out, idx) in zip(dms, cases, got):
        rout = torch.zeros(B * O, device=dev)
        ridx = torch.empty(B * T, dtype=torch.int32, device=dev)
        _native.check(L.spiky_lut_forward_step(dm._h, _p(W), B, _p(x), _p(anchors), _p(rout), _p(ridx),
                                               ctypes.c_float(0.0), None, None, stream))
        torch.cuda.synchronize()
        assert torch.equal(idx.cpu(), ridx.cpu())
        assert torch.equal(out.cpu().view(torch.int32), rout.cpu().view(torch.int32))
