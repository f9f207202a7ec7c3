"""LUT layer forward+backward benchmark (BASELINE config 3 by default).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3|1|4] [--no-cpu-baseline]

A step is one forward + backward of the dense LUT layer through its autograd
function (LUTForwardFN via LUTLayer.__call__ and Tensor.backward) on one batch
of synthetic, HBM-resident input: the same work the reference's
LUTLayer.forward/backward_step perform (check_detectors, fill_outputs,
propagate_through_detectors, gather_w_gradients) plus the layer's own
allocations.  Per-kernel GPU times come from HIP events recorded on the launch
stream inside the timed region.  The CPU baseline is the C oracle (a serial
restatement of the reference's CPU path) timed on one host core on a bounded
batch of the same workload.

Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0  # MI355X HBM3E peak
PEAK_FP64_TFLOPS = 78.6  # MI355X fp64 (vector and matrix)

CONFIGS = {
    # name: (B, I, T, Nc, O, x_dist, cpu_sample_B)
    1: (64, 784, 256, 6, 10, "uniform", 64),
    3: (1024, 4096, 8192, 8, 1024, "normal", 256),
}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def g_model_bytes(B, I, T, Nc, O, w=4):
    """Algorithmic bytes per kernel family, gather model (the embedding-bag
    convention): every logical row access counts once per use, with no credit
    for cache or LDS reuse."""
    return {
        "check_detectors": B * I * 4 + T * Nc * 8 + B * T * 12,
        "fill_outputs_fc": B * T * O * w + B * O * 4,
        "propagate_fc": 2 * B * T * O * 4 + B * O * 4 + B * T * 12 + B * I * 4 + T * Nc * 8,
        "gather_w_gradients_fc": 2 * B * T * O * 4,
    }


def unique_bytes(B, I, T, Nc, O, w=4):
    """Unique bytes per kernel family: what one launch must move across HBM at
    least, each tensor once.  Per unit: the detector check reads 4 B per input
    element and 8 B per anchor pair and writes 12 B per (sample, table); the
    forward reads every table byte and 4 B of index per (sample, table) and
    updates 4 B per output; the propagate reads every table byte, 4 B of output
    gradient per output and 12 B per (sample, table), and updates 4 B per input
    gradient element; the weight gradient writes every gradient byte and reads
    the output gradient and the indices."""
    E = 1 << Nc
    tables = T * E * O * w
    return {
        "check_detectors": B * I * 4 + T * Nc * 8 + B * T * 12,
        "fill_outputs_fc": tables + B * T * 4 + 2 * B * O * 4,
        "propagate_fc": tables + B * O * 4 + B * T * 12 + T * Nc * 8 + 2 * B * I * 4,
        "gather_w_gradients_fc": T * E * O * 4 + B * O * 4 + B * T * 4,
    }


def compulsory_bytes(B, I, T, Nc, O):
    """Unique bytes a step must move at least: the tables read in forward and
    backward, and the weight gradient written once."""
    E = 1 << Nc
    return 3 * T * E * O * 4 + 2 * B * I * 4 + 2 * B * O * 4 + B * T * 12


def source_digest():
    """sha256 (first 16 hex digits) of the HIP sources the library is built
    from; counter summaries record the digest they were taken at."""
    import hashlib
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "spiky_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h")):
            with open(os.path.join(csrc, name), "rb") as f:
                h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class pinned_core:
    """Runs the enclosed CPU baseline on one host core (the reference CPU path
    is single-threaded), restoring the affinity afterwards."""

    def __enter__(self):
        self.saved = os.sched_getaffinity(0)
        self.core = min(self.saved)
        os.sched_setaffinity(0, {self.core})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.saved)
        return False


def make_anchors(T, I, Nc, seed, device):
    """Nc distinct (a1, a2) pairs per table: 2*Nc distinct inputs drawn without
    replacement per table, paired in order."""
    import torch
    g = torch.Generator(device=device).manual_seed(seed)
    perm = torch.rand(T, I, device=device, generator=g).argsort(dim=1)[:, :2 * Nc]
    return perm.to(torch.int32).reshape(-1).contiguous()


def load_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy-kernel
    calibration factor), with the source digest the summary was taken at.
    Lines read "<kernel> <bytes>" and "# sources <digest>".  Returns
    (bytes or None, digest or None)."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_config{config}.txt")
    if not os.path.exists(path):
        return None, None
    value = digest = None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if line.startswith("# sources") and len(parts) == 3:
                digest = parts[2]
            elif len(parts) == 2 and parts[0] == kernel and not line.startswith("#"):
                value = float(parts[1])
    return value, digest


def traffic_fields(key, config, ms):
    """roofline.traffic and its rate: measured HBM bytes per launch of family
    `key` (or per step, key "step") from profiles/hbm_traffic_config<N>.txt,
    null when that summary was taken at other kernel sources."""
    traffic, digest = load_traffic(key, config)
    stale = traffic is not None and digest != source_digest()
    if stale:
        traffic = None
    return {"traffic": traffic, "traffic_source_digest": digest, "traffic_stale": stale,
            "traffic_gbs": round(traffic / (ms * 1e-3) / 1e9, 1) if traffic else None}


def calibrate_copy(mib):
    """A plain device-to-device copy of `mib` MiB, five times: the known-size
    kernel the FETCH_SIZE / WRITE_SIZE counters are scaled against."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {mib} MiB x5 ({n * 4} bytes read and written per copy)")


def cpu_baseline(x, anchors, W, go, B_full, I, T, Nc, O, sample_B):
    """Times the C oracle on one host core over the first sample_B samples:
    forward (indices + gather-sum) and backward (propagate + weight gradient),
    including the caller-side zero-fill of out, x_grad and w_grad that the
    reference's LUTLayer performs (LUTLayer.py:631,851,864)."""
    import numpy as np
    import oracle
    E = 1 << Nc
    log(f"cpu baseline: copying tables to host ({W.numel() * 4 / 1e9:.1f} GB)")
    Wn = W.cpu().numpy()
    xn = x[:sample_B * I].cpu().numpy()
    gn = go[:sample_B * O].cpu().numpy()
    an = anchors.cpu().numpy()
    wg = np.empty(T * E * O, np.float32)
    times = []
    zero_fill = []
    with pinned_core() as pin:
        core = pin.core
        for rep in range(3):
            t0 = time.perf_counter()
            out = np.zeros(sample_B * O, np.float32)
            idx, md, mi = oracle.check_detectors(xn, an, sample_B, I, T, Nc)
            oracle.fill_outputs_fc(Wn, idx, sample_B, O, T, E, out=out)
            xg = np.zeros(sample_B * I, np.float32)
            tz = time.perf_counter()
            wg.fill(0.0)
            zero_fill.append(time.perf_counter() - tz)
            oracle.propagate_fc(Wn, gn, idx, md, mi, an, sample_B, I, O, T, Nc, E, x_grad=xg)
            oracle.gather_wgrad_fc(gn, idx, wg, sample_B, O, T, E)
            dt = time.perf_counter() - t0
            log(f"cpu baseline rep {rep}: {dt:.2f} s")
            if rep > 0:
                times.append(dt)
    med = float(np.median(times))
    return {
        "value": sample_B / med,
        "unit": "samples/s",
        "cores": 1,
        "kind": "port",
        "cpu": f"{cpu_model()} (pinned to core {core})",
        "sample": (f"config workload at batch {sample_B} of {B_full} (same tables, anchors, inputs); "
                   f"median of 2 timed steps after 1 warm-up; step {med:.3f} s of which w_grad "
                   f"zero-fill {float(np.median(zero_fill[1:])):.3f} s"),
    }


PROJ = dict(B=128, cpu_reps=121)


def build_projection_stack(device, seed=1):
    """BASELINE config 2 on this build's ProjectionLUTLayer: 28x28 input;
    layer 1 a 12x12 grid (stride 2) of 5x5 receptive fields, 32 tables of 5
    anchor pairs per group, each projecting onto a 4x4 patch (16 channels) of
    a 48x48 map; layer 2 a 5x5 grid (stride 2 positions = 8 pixels) of 3x3-
    position (12x12-pixel) windows of that map, 64 tables of 6 pairs per group,
    each onto 4x8 = 32 channels of a 20x40 map; a dense head of 128 tables,
    6 pairs, 10 outputs."""
    from spiky_amd import LUTLayer, ProjectionLUTLayer
    from spiky_amd.util.synapse_growth import PointSamplingPolicy, PointSamplingType
    l1 = ProjectionLUTLayer((28, 28), (48, 48), 5, 144, 32, (5, 5), (4, 4),
                            detectors_sampling_policy=PointSamplingPolicy(
                                PointSamplingType.Grid, pad_h=2.0, pad_w=2.0, grid_h=12, grid_w=12,
                                stride_h=2, stride_w=2),
                            random_seed=seed, device=device)
    l2 = ProjectionLUTLayer((48, 48), (20, 40), 6, 25, 64, (12, 12), (4, 8),
                            detectors_sampling_policy=PointSamplingPolicy(
                                PointSamplingType.Grid, pad_h=6.0, pad_w=6.0, grid_h=5, grid_w=5,
                                stride_h=8, stride_w=8),
                            random_seed=seed + 1, device=device)
    head = LUTLayer(800, 6, 128, 10, random_seed=seed + 2, device=device)
    return l1, l2, head


def bench_projection(args):
    """the sparse ProjectionLUTLayer stack forward and
    backward at batch 128 on 80%-zero uniform images."""
    import torch
    import numpy as np
    B = PROJ["B"]
    dev = torch.device("cuda:0")
    log("config 2: ProjectionLUTLayer stack")
    l1, l2, head = build_projection_stack(dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    with torch.no_grad():
        for layer in (l1, l2, head):
            layer._weights.normal_(0.0, 0.01, generator=gen)
    gx = torch.Generator(device=dev).manual_seed(0)
    x = torch.rand(B, 1, 28, 28, device=dev, generator=gx)
    x = (x * (torch.rand(B, 1, 28, 28, device=dev, generator=gx) > 0.8)).requires_grad_(True)
    g = torch.randn(B, 1, 10, device=dev, generator=gx)
    params = [l1._weights, l2._weights, head._weights]

    def step():
        for p_ in params:
            p_.grad = None
        x.grad = None
        y1 = l1(x)
        y2 = l2(y1.reshape(B, 1, 48, 48))
        out = head(y2.reshape(B, 1, 800))
        out.backward(g)

    log("warmup")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    # the same eager step with the backward run on the calling thread instead
    # of the device's autograd worker thread (a PyTorch switch; same kernels)
    with torch.autograd.set_multithreading_enabled(False):
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ms_one_thread = (time.perf_counter() - t0) * 1e3 / args.steps
    log(f"backward on the calling thread: {ms_one_thread:.3f} ms/step")
    # per-family times in a separate pass: the events around each of the
    # stack's 15 launches would otherwise weigh on a sub-millisecond step
    dms = [l1._lut_dm, l2._lut_dm, head._lut_dm]
    for d in dms:
        d.get_kernel_times(reset=True)
        d.set_kernel_timing(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ktimes = {}
    for name, d in zip(("layer1", "layer2", "head"), dms):
        d.set_kernel_timing(False)
        for k, (cnt, tot) in d.get_kernel_times(reset=True).items():
            ktimes[f"{name}.{k}"] = tot / max(cnt, 1)
    log(f"{ms:.3f} ms/step; kernels {ktimes}")
    graph_ms = projection_graph_ms(step, args.steps)
    log(f"graph replay: {graph_ms:.3f} ms/step")
    roofline = projection_roofline(l1, l2, head, x.detach(), B, ktimes)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_projection(l1, l2, head, x.detach(), g, B, PROJ["cpu_reps"])
    res = {
        "metric": "ProjectionLUTLayer stack fwd+bwd samples/sec (BASELINE config 2)",
        "value": round(B / (ms / 1e3), 1),
        "unit": "samples/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 (fp64 partial sums)",
        "data": "synthetic (uniform [0,1) 28x28 images with 80% of pixels zeroed, N(0,0.01) tables, N(0,1) grads)",
        "config": {"workload": "BASELINE config 2: sparse ProjectionLUTLayer stack fwd+bwd", "batch": B,
                   "layer1": "28x28 -> 48x48, 144 groups x 32 tables, 5 pairs, 5x5 fields, 16 targets",
                   "layer2": "48x48 -> 20x40, 25 groups x 64 tables, 6 pairs, 12x12 fields, 32 targets",
                   "head": "800 -> 10, 128 tables, 6 pairs", "parallelism": "single GPU"},
        "eager_backward_on_calling_thread": {
            "ms_per_step": round(ms_one_thread, 4), "value": round(B / (ms_one_thread / 1e3), 1),
            "unit": "samples/s",
            "note": "the eager step under torch.autograd.set_multithreading_enabled(False): the host-bound "
                    "step saves the hand-over to the device's autograd thread"},
        "graph_replay": {"ms_per_step": round(graph_ms, 4), "value": round(B / (graph_ms / 1e3), 1),
                         "unit": "samples/s",
                         "note": "the same step captured once in a HIP graph (torch.cuda.CUDAGraph) and "
                                 "replayed: the same kernels without the host's per-launch work"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


def projection_graph_ms(step, steps):
    """Milliseconds per step of `step` captured in a HIP graph and replayed
    (warmed up on a side stream first, as graph capture requires)."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def projection_roofline(l1, l2, head, x, B, ktimes):
    """Roofline of config 2's dominant kernel family, with bytes from the built
    CSR.  Each (sample, table) lookup of a sparse layer reaches the synapses
    of one lookup neuron: G model = 4 bytes x those synapses x 5 (forward
    read, main and flipped reads in the propagate, read-modify-write of the
    weight gradient) plus 12 bytes of index and margins; unique bytes = every
    synapse weight (forward and propagate families) or weight-gradient word
    (weight-gradient family) once, plus the activations."""
    import numpy as np
    import torch
    layers = {"layer1": (l1, 784, 2304, 5), "layer2": (l2, 2304, 800, 6)}
    # the lookup indices of this input, from the layers' own forward
    with torch.no_grad():
        r1 = l1.forward_step(x.reshape(B, 1, 28, 28))
        r2 = l2.forward_step(r1[0].reshape(B, 1, 48, 48))
    idxs = {"layer1": r1[1].cpu().numpy(), "layer2": r2[1].cpu().numpy()}
    fams = {}
    for name, (layer, I, O, Nc) in layers.items():
        offs, tg = layer._lut_dm.lookup_connectivity()
        T = layer.n_detectors()
        neuron = (np.arange(T)[None, :] * (1 << Nc) + idxs[name].reshape(B, T)).reshape(-1)
        hits = int(np.sum(offs[neuron + 1] - offs[neuron]))
        n_syn = int(tg.size)
        side = B * I * 4 + B * O * 4 + B * T * 12
        fams[f"{name}.fill_outputs_sparse"] = (n_syn * 4 + side, hits * 4 + side)
        fams[f"{name}.propagate_sparse"] = (n_syn * 4 + side + B * I * 4, 2 * hits * 4 + side)
        fams[f"{name}.gather_w_gradients_sparse"] = (n_syn * 4 + B * O * 4 + B * T * 4, 2 * hits * 4)
    known = {k: v for k, v in ktimes.items() if k in fams}
    if not known:
        return None
    dom = max(known, key=known.get)
    ms = known[dom]
    ub, gb = fams[dom]
    return {"bound": "hbm", "kernel": dom, "achieved": round(ub / (ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
            "unit": "GB/s", "frac": round(ub / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "traffic": None,
            "algorithmic_bytes_per_launch": ub, "ms_per_launch": round(ms, 4),
            "g_model": {"bytes_per_launch": gb, "frac": round(gb / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
            "kernels": {k: round(v, 4) for k, v in ktimes.items()}}


def cpu_projection(l1, l2, head, x, g, B, reps):
    """The C oracle over the same stack: forward through the three layers, then
    backward (input and weight gradients of each)."""
    import numpy as np
    import oracle

    def sparse_parts(layer):
        offs, tg = layer._lut_dm.lookup_connectivity()
        return (layer._weights.detach().cpu().numpy(), layer._detector_anchors.cpu().numpy(), offs, tg,
                layer._lut_dm.get_max_forward_groups_per_neuron())

    p1, p2 = sparse_parts(l1), sparse_parts(l2)
    Wh, ah = head._weights.detach().cpu().numpy(), head._detector_anchors.cpu().numpy()
    xn, gn = x.cpu().numpy().reshape(-1), g.cpu().numpy().reshape(-1)
    times = []
    pin = pinned_core()
    pin.__enter__()
    for rep in range(reps):
        t0 = time.perf_counter()
        acts = [xn]
        saved = []
        for (W, an, offs, tg, _), (I, O, T, Nc) in ((p1, (784, 2304, 4608, 5)), (p2, (2304, 800, 1600, 6))):
            idx, md, mi = oracle.check_detectors(acts[-1], an, B, I, T, Nc)
            saved.append((idx, md, mi))
            acts.append(oracle.fill_outputs_sparse(W, idx, offs, tg, B, O, T, 1 << Nc))
        hidx, hmd, hmi = oracle.check_detectors(acts[-1], ah, B, 800, 128, 6)
        oracle.fill_outputs_fc(Wh, hidx, B, 10, 128, 64)
        grad = oracle.propagate_fc(Wh, gn, hidx, hmd, hmi, ah, B, 800, 10, 128, 6, 64)
        oracle.gather_wgrad_fc(gn, hidx, np.zeros(Wh.size, np.float32), B, 10, 128, 64)
        for (W, an, offs, tg, maxg), (idx, md, mi), (I, O, T, Nc) in (
                (p2, saved[1], (2304, 800, 1600, 6)), (p1, saved[0], (784, 2304, 4608, 5))):
            oracle.gather_wgrad_sparse(grad, idx, offs, tg, np.zeros(W.size, np.float32), B, O, T, 1 << Nc)
            grad = oracle.propagate_sparse(W, grad, idx, md, mi, an, offs, tg, B, I, O, T, Nc, 1 << Nc, 32, maxg)
        dt = time.perf_counter() - t0
        if rep > 0:
            times.append(dt)
    pin.__exit__(None, None, None)
    med = float(np.median(times))
    return {"value": B / med, "unit": "samples/s", "cores": 1, "kind": "port",
            "cpu": f"{cpu_model()} (pinned to core {pin.core})",
            "sample": f"the whole config-2 step at batch {B}; median of {reps - 1} after 1 warm-up; step {med:.3f} s"}


INT8 = dict(B=4096, I=4096, T=8192, Nc=8, O=1024, int_rescaler=0.001, cpu_B=2048)


def int8_unique_bytes(B, I, T, Nc, O):
    """Unique bytes per family of the int8 forward: the detector check reads
    x and the anchors and writes the indices; the gather-sum reads the int8
    tables and scales once and the indices, and updates the output."""
    E = 1 << Nc
    return {"check_detectors": B * I * 4 + T * Nc * 8 + B * T * 4,
            "fill_outputs_fc_i8": T * E * O + T * 4 + B * T * 4 + 2 * B * O * 4}


def bench_int8(args):
    """the config-3 layer with int8 tables (uniform in
    [-127, 127]) and one fp32 scale per table (uniform [0.001, 0.01]),
    int32 summation (LUTDataManagerI), inference forward at batch 4096:
    indices plus the gather-sum of scale[t] * q rows."""
    import torch
    import numpy as np
    from spiky_amd import LUTDataManagerI
    c = INT8
    B, I, T, Nc, O = c["B"], c["I"], c["T"], c["Nc"], c["O"]
    E = 1 << Nc
    dev = torch.device("cuda:0")
    log(f"config 4: int8 tables, B={B} I={I} T={T} Nc={Nc} O={O}")
    anchors = make_anchors(T, I, Nc, 1, dev)
    gq = torch.Generator(device=dev).manual_seed(4)
    q8 = torch.randint(-127, 128, (T * E * O,), device=dev, generator=gq, dtype=torch.int8)
    scales = torch.rand(T, device=dev, generator=gq) * 0.009 + 0.001
    gx = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(B * I, device=dev, generator=gx)
    dm = LUTDataManagerI(I, O, T, Nc, 1, 0, 0, 32, 32, c["int_rescaler"])
    dm.register_synapse_meta(1.0, -1.0, 1.0, 0.0, 0.0)
    dm.initialize_neurons(True)
    dm.to_device(0)
    out = torch.empty(B * O, device=dev)
    idx = torch.empty(B * T, dtype=torch.int32, device=dev)

    def step():
        out.zero_()  # the caller's zeroed output (LUTLayer.py:631)
        dm.forward_step_i8(q8, scales, B, x, anchors, out, idx)

    log("warmup")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    dm.get_kernel_times(reset=True)
    dm.set_kernel_timing(True)
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    dm.set_kernel_timing(False)
    ktimes = dm.get_kernel_times(reset=True)
    log(f"{ms:.3f} ms/step; kernels {ktimes}")
    gb = {"check_detectors": B * I * 4 + T * Nc * 8 + B * T * 4,
          "fill_outputs_fc_i8": B * T * O * 1 + T * 4 + B * O * 4}
    ub = int8_unique_bytes(B, I, T, Nc, O)
    dom = max(ktimes.items(), key=lambda kv: kv[1][1])[0]
    dom_ms = ktimes[dom][1] / ktimes[dom][0]
    achieved = ub[dom] / (dom_ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        import oracle
        sb = c["cpu_B"]
        log(f"cpu baseline: copying int8 tables to host ({q8.numel() / 1e9:.1f} GB)")
        qn, scn = q8.cpu().numpy(), scales.cpu().numpy()
        xn, an = x[:sb * I].cpu().numpy(), anchors.cpu().numpy()
        times = []
        with pinned_core() as pin:
            for rep in range(3):
                t1 = time.perf_counter()
                o = np.zeros(sb * O, np.float32)
                ridx = oracle.check_detectors(xn, an, sb, I, T, Nc, train=False)
                oracle.fill_outputs_fc(None, ridx, sb, O, T, E, out=o, q8=qn, scales=scn, int_mode=True,
                                       int_rescaler=c["int_rescaler"])
                oracle.convert_int_to_float(o, c["int_rescaler"])
                dt = time.perf_counter() - t1
                log(f"cpu baseline rep {rep}: {dt:.2f} s")
                if rep > 0:
                    times.append(dt)
        med = float(np.median(times))
        cpu = {"value": sb / med, "unit": "samples/s", "cores": 1, "kind": "port",
               "cpu": f"{cpu_model()} (pinned to core {pin.core})",
               "sample": f"config-4 workload at batch {sb} of {B}; median of 2 after 1 warm-up; step {med:.3f} s"}
    res = {
        "metric": "int8 LUT forward samples/sec at 8192 tables (BASELINE config 4)",
        "value": round(B / (ms / 1e3), 1),
        "unit": "samples/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 tables, int32 accumulators",
        "data": "synthetic (seeded N(0,1) inputs, int8 tables uniform [-127,127], scales uniform [0.001,0.01])",
        "config": {"workload": "BASELINE config 4: int8 LUT layer inference forward", "batch": B,
                   "n_inputs": I, "n_tables": T, "anchors_per_table": Nc, "n_outputs": O,
                   "table_bytes": T * E * O, "int_rescaler": c["int_rescaler"], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4), **traffic_fields(dom, 4, dom_ms),
                     "algorithmic_bytes_per_launch": ub[dom], "ms_per_launch": round(dom_ms, 4),
                     "g_model": {"bytes_per_launch": gb[dom],
                                 "frac": round(gb[dom] / (dom_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
                     "kernels": {k: round(v[1] / v[0], 4) for k, v in ktimes.items()}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


TRANSFORMER = dict(vocab_size=256, embedding_dim=256, context_size=256, positional_dim=4, num_layers=4,
                   num_heads=4, n_detectors=16, n_anchors_per_detector=8,
                   n_anchors_per_detector_attention=6)
TRANSFORMER_BATCH = 32


def transformer_g_bytes(B, cfg):
    """G-model bytes of one forward + backward of the config-5 transformer:
    every causal pair reads one attention row forward and its main and flipped
    rows backward (plus the row read-modify-write of the weight gradient);
    feed-forward and unembedding layers as in g_model_bytes over B*S rows."""
    S, E, V = cfg["context_size"], cfg["embedding_dim"], cfg["vocab_size"]
    T_att = cfg["n_detectors"] * cfg["num_heads"]
    pairs = S * (S - 1) // 2
    att = B * pairs * T_att * E * 4 * (1 + 2 + 2)
    fc = lambda O: sum(g_model_bytes(B * S, E, cfg["n_detectors"], cfg["n_anchors_per_detector"], O).values())
    return cfg["num_layers"] * (att + fc(E)) + fc(V)


def transformer_unique_bytes(B, model):
    """Unique bytes of one config-5 step: every LUT table read in the forward
    and in the backward and its weight gradient written once, plus each LUT
    layer's input and output activations and their gradients once."""
    S, E = model.context_size, model.embedding_dim if isinstance(model.embedding_dim, int) else \
        model.embedding_dim[0] * model.embedding_dim[1]
    total = 0
    for layer in model._lut_layers():
        total += 3 * layer._weights.numel() * 4
        total += 2 * B * S * (layer._n_inputs + layer._n_outputs) * 4
    return total


def cpu_transformer(model, tokens, targets):
    """The C oracle chained as the model runs (one sequence): embedding, per
    block the sequence-concat attention LUT plus residual and the feed-forward
    LUT plus residual, the unembedding LUT, the cross-entropy gradient, then
    the backward through the same layers (input and weight gradients of every
    LUT, positional-embedding gradients).  One host core, median of 2 after a
    warm-up."""
    import numpy as np
    import oracle
    B, S = tokens.shape
    V = model.vocab_size
    E = model.embedding_dim
    blocks = []
    for b in model.layers:
        att, ffn = b["attention_lut"], b["ffn"]
        blocks.append((att, ffn, att._weights.detach().cpu().numpy(), att._detector_anchors.cpu().numpy(),
                       att._positional_embeddings.detach().cpu().numpy(), ffn._weights.detach().cpu().numpy(),
                       ffn._detector_anchors.cpu().numpy()))
    un = model.unembedder
    Wu, au = un._weights.detach().cpu().numpy(), un._detector_anchors.cpu().numpy()
    emb = model.token_embedder.weight.detach().cpu().numpy()
    tk, tg = tokens.cpu().numpy(), targets.cpu().numpy().reshape(-1)

    def one_step():
        z = emb[tk].astype(np.float32).reshape(-1)
        saved = []
        for att, ffn, Wa, aa, pe, Wf, af in blocks:
            T, Nc, Npe = att._n_detectors, att._n_anchors_per_detector, att._positional_dim
            idx, md, mi = oracle.check_detectors(z, aa, B * S, E, T, Nc)
            pidx, pmd, pmi = oracle.check_pe(pe, S, T, Npe)
            a = oracle.fill_outputs_seq(Wa, idx, pidx, B, E, T, S, Nc, Npe)
            saved.append(("att", att, Wa, aa, (idx, md, mi, pidx, pmd, pmi)))
            z = z + a
            Tf, Ncf = ffn._n_detectors, ffn._n_anchors_per_detector
            fi, fmd, fmi = oracle.check_detectors(z, af, B * S, E, Tf, Ncf)
            z = z + oracle.fill_outputs_fc(Wf, fi, B * S, E, Tf, 1 << Ncf)
            saved.append(("ffn", ffn, Wf, af, (fi, fmd, fmi)))
        Tu, Ncu = un._n_detectors, un._n_anchors_per_detector
        ui, umd, umi = oracle.check_detectors(z, au, B * S, E, Tu, Ncu)
        logits = oracle.fill_outputs_fc(Wu, ui, B * S, V, Tu, 1 << Ncu).reshape(B * S, V).astype(np.float64)
        p = np.exp(logits - logits.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        p[np.arange(B * S), tg] -= 1.0
        grad = (p / (B * S)).astype(np.float32).reshape(-1)
        wg = np.zeros(Wu.size, np.float32)
        oracle.gather_wgrad_fc(grad, ui, wg, B * S, V, Tu, 1 << Ncu)
        grad = oracle.propagate_fc(Wu, grad, ui, umd, umi, au, B * S, E, V, Tu, Ncu, 1 << Ncu)
        for kind, layer, W, an, keys in reversed(saved):
            T, Nc = layer._n_detectors, layer._n_anchors_per_detector
            wg = np.zeros(W.size, np.float32)
            if kind == "ffn":
                fi, fmd, fmi = keys
                oracle.gather_wgrad_fc(grad, fi, wg, B * S, E, T, 1 << Nc)
                xg = oracle.propagate_fc(W, grad, fi, fmd, fmi, an, B * S, E, E, T, Nc, 1 << Nc)
            else:
                idx, md, mi, pidx, pmd, pmi = keys
                Npe = layer._positional_dim
                oracle.gather_wgrad_seq(grad, idx, pidx, wg, B, E, T, S, Nc, Npe)
                xg, _ = oracle.propagate_seq(W, grad, idx, md, mi, pidx, pmd, pmi, an, B, E, E, T, S, Nc, Npe)
            grad = (grad + xg).astype(np.float32)

    times = []
    with pinned_core() as pin:
        for rep in range(3):
            t0 = time.perf_counter()
            one_step()
            dt = time.perf_counter() - t0
            log(f"cpu baseline rep {rep}: {dt:.2f} s")
            if rep > 0:
                times.append(dt)
    med = float(np.median(times))
    return {"value": B / med, "unit": "samples/s", "cores": 1, "kind": "port",
            "cpu": f"{cpu_model()} (pinned to core {pin.core})",
            "sample": f"one sequence of the config-5 step (forward, cross-entropy gradient, backward) "
                      f"through the C oracle; median of 2 after 1 warm-up; step {med:.2f} s"}


def bench_transformer(args):
    """LUTTransformer forward + cross-entropy + backward on
    random byte tokens with next-token targets."""
    import torch
    import torch.nn.functional as F
    from spiky_amd import LUTTransformer
    dev = torch.device("cuda:0")
    cfg = TRANSFORMER
    B, S, V = TRANSFORMER_BATCH, cfg["context_size"], cfg["vocab_size"]
    log(f"config 5: LUTTransformer {cfg}, batch {B}")
    model = LUTTransformer(**cfg, device=dev, seed=1)
    gen = torch.Generator(device=dev).manual_seed(2)
    with torch.no_grad():
        for layer in model._lut_layers():
            layer._weights.normal_(0.0, 0.01, generator=gen)
    gt = torch.Generator(device=dev).manual_seed(0)
    stream = torch.randint(0, V, (B, S + 1), device=dev, generator=gt)
    tokens, targets = stream[:, :S].contiguous(), stream[:, 1:].contiguous()
    params = [l._weights for l in model._lut_layers()] + \
             [b["attention_lut"]._positional_embeddings for b in model.layers]

    def step():
        for p in params:
            p.grad = None
        logits = model(tokens)
        loss = F.cross_entropy(logits.reshape(-1, V), targets.reshape(-1))
        loss.backward()

    log("warmup")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    g = transformer_g_bytes(B, cfg)
    u = transformer_unique_bytes(B, model)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_transformer(model, tokens[:1], targets[:1])
    res = {
        "metric": "LUTTransformer fwd+bwd samples/sec (BASELINE config 5)",
        "value": round(B / (ms / 1e3), 2),
        "unit": "samples/s",
        "tokens_per_s": round(B * S / (ms / 1e3), 1),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32 (fp64 partial sums)",
        "data": "synthetic (uniform random byte tokens, next-token targets, N(0,0.01) tables)",
        "config": {"workload": "BASELINE config 5: LUTTransformer block stack fwd+bwd", "batch": B, **cfg},
        "roofline": {"bound": "hbm", "achieved": round(u / (ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(u / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                     **traffic_fields("step", 5, ms), "algorithmic_bytes_per_step": u,
                     "scope": "whole step, unique bytes (every table read forward and backward, every "
                              "weight gradient written once, activations)",
                     "g_model": {"bytes_per_step": g, "frac": round(g / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


PRODUCT = dict(batch=32, seq_len=256, n_inputs=256, n_detectors=64, n_anchors=6, n_outputs=256,
               positional_dim=4, cpu_batch=2)


def product_flops(B, S, T, Nc, O):
    """fp64 FMA flops of the three count products of one product-mode fwd+bwd
    (out += Cnt.W, P = G.W^T, W_grad += Cnt^T.G), each B*S x T*2^Nc x O."""
    return 3 * 2 * B * S * (T << Nc) * O


def bench_product(args):
    """Product-mode LUT layer (concatenation_product=False) forward + backward
    at the attention shape of BASELINE config 5: 32 sequences of 256 tokens,
    d_model 256, 16 detectors x 4 heads, 6 anchors (64-row tables) over the
    virtual row [x_i | x_j | pe] with positional_dim 4, Dense weight gradient."""
    import torch
    from spiky_amd import LUTLayer
    dev = torch.device("cuda:0")
    c = PRODUCT
    B, S, n, T, Nc, O, pd = (c[k] for k in ("batch", "seq_len", "n_inputs", "n_detectors", "n_anchors",
                                             "n_outputs", "positional_dim"))
    log(f"product: B={B} S={S} n={n} T={T} Nc={Nc} O={O} pd={pd}")
    layer = LUTLayer(n, Nc, T, O, sequence_length=S, concatenation_product=False, positional_dim=pd,
                     random_seed=1, device=dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.01, generator=gen)
    x = torch.randn(B, S, n, device=dev, generator=gen).requires_grad_(True)
    go = torch.randn(B, S, O, device=dev, generator=gen)

    def step():
        x.grad = None
        layer._weights.grad = None
        layer._positional_embeddings.grad = None
        layer(x).backward(go)

    log("warmup")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    fl = product_flops(B, S, T, Nc, O)
    lookups = 2 * B * (S * (S - 1) // 2) * T
    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np
        import oracle
        cb = c["cpu_batch"]
        xs = x.detach()[:cb].cpu().numpy().reshape(-1)
        W = layer._weights.detach().cpu().numpy()
        anc = layer._detector_anchors.cpu().numpy()
        pe = layer._prepare_positional_embeddings().detach().cpu().numpy()
        g = go[:cb].cpu().numpy().reshape(-1)
        geo = (cb, S, n, n, pd, T, Nc, O)
        t0 = time.perf_counter()
        oracle.fill_outputs_product(xs, xs, pe, anc, W, *geo)
        oracle.propagate_product(xs, xs, pe, anc, W, g, *geo, w_grad=np.zeros(W.size, np.float32))
        sec = time.perf_counter() - t0
        cpu = {"value": round(cb / sec, 4), "unit": "samples/s", "cores": 1, "kind": "port",
               "sample": f"C restatement of the reference's CPU product path (serial, 1 thread) on {cb} of "
                         f"the {B} sequences, forward + backward: {sec:.2f} s"}
    res = {
        "metric": "product-mode LUT layer fwd+bwd samples/sec (config-5 attention shape)",
        "value": round(B / (ms / 1e3), 2), "unit": "samples/s",
        "pair_lookups_per_s": round(lookups / (ms / 1e3), 1),
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64 (fp32 I/O)",
        "data": "synthetic (N(0,1) inputs and upstream grads, N(0,0.01) tables)",
        "config": {"workload": "product-mode LUT layer fwd+bwd, config-5 attention shape", **c},
        "roofline": {"bound": "mfma", "achieved": round(fl / (ms * 1e-3) / 1e12, 2), "peak": PEAK_FP64_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(fl / (ms * 1e-3) / 1e12 / PEAK_FP64_TFLOPS, 4),
                     "traffic": None, "flops_per_step": fl, "scope": "whole step, fp64 count products"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


DENSIFY = dict(words=1 << 28, densities=(0.01, 0.1, 0.5), cpu_words=1 << 25)


def bench_densify(args):
    """The Sparse policy's dense -> sparse export (DenseToSparseConverter,
    lut_densify.hip) on a 1 GiB fp32 gradient at three densities, with
    erase_input=True as LUTLayer uses it.  HBM bytes per call: the source read
    twice (count, then compaction), 12 bytes per kept word (int64 index + value)
    and 16 per erased quad."""
    import torch
    from spiky_amd.util.torch_utils import DenseToSparseConverter
    dev = torch.device("cuda:0")
    n = DENSIFY["words"]
    g = torch.Generator(device=dev).manual_seed(0)
    conv = DenseToSparseConverter()
    rows = []
    for dens in DENSIFY["densities"]:
        src0 = torch.randn(n, device=dev, generator=g)
        src0[torch.rand(n, device=dev, generator=g) >= dens] = 0.0
        nnz = int(torch.count_nonzero(src0))
        quads = int(torch.count_nonzero(src0.view(-1, 4).abs().sum(1)))
        bufs = (torch.empty(nnz, dtype=torch.int64, device=dev), torch.empty(nnz, device=dev))
        src = torch.empty_like(src0)
        times = []
        for it in range(args.warmup + args.steps):
            src.copy_(src0)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            conv.dense_to_sparse_32(src, True, bufs, decouple=False)
            b.record()
            torch.cuda.synchronize()
            if it >= args.warmup:
                times.append(a.elapsed_time(b))
        ms = float(sorted(times)[len(times) // 2])
        traffic = 2 * 4 * n + 12 * nnz + 16 * quads
        rows.append({"density": dens, "nnz": nnz, "ms": round(ms, 4),
                     "gb_per_s": round(traffic / ms / 1e6, 1)})
        log(f"densify density {dens}: {ms:.3f} ms, {traffic / ms / 1e6:.0f} GB/s")
    main_row = rows[1]
    cpu = None
    if not args.no_cpu_baseline:
        import numpy as np
        import oracle
        m = DENSIFY["cpu_words"]
        rng = np.random.default_rng(0)
        a = rng.standard_normal(m).astype(np.float32)
        a[rng.random(m) >= DENSIFY["densities"][1]] = 0.0
        t = []
        for _ in range(5):
            t0 = time.perf_counter()
            oracle.dense_to_sparse_32(a)
            t.append(time.perf_counter() - t0)
        med = float(np.median(t[1:]))
        cpu = {"value": round(m * 4 / med / 1e9, 2), "unit": "GB/s of source", "cores": 1, "kind": "port",
               "sample": f"numpy restatement on {m} words at density 0.1; median of 4 after 1 warm-up; "
                         f"{med:.3f} s per call"}
    out = {
        "metric": "dense_to_sparse_32 source GB/s (GradientType.Sparse export, density 0.1)",
        "value": round(n * 4 / main_row["ms"] / 1e6, 1), "unit": "GB/s of source", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": main_row["ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32",
        "data": "synthetic (N(0,1) fp32 words, zeroed at random to the density)",
        "config": {"workload": "dense -> sparse COO of a 1 GiB fp32 gradient, erase_input=True",
                   "words": n, "densities": rows},
        "roofline": {"bound": "hbm", "achieved": main_row["gb_per_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(main_row["gb_per_s"] / PEAK_HBM_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


# Kernels of each C-ABI launch family (one call = these kernels in order), by
# configuration: the trace and counter summaries sum them per family.
FAMILIES = {
    3: {"check_detectors": ["k_check_detectors_lds"],
        "fill_outputs_fc": ["k_transpose_idx", "k_fill_tm_dma", "k_fill_commit"],
        "propagate_fc": ["k_transpose_keys4", "k_propagate_units", "k_propagate_scatter"],
        "gather_w_gradients_fc": ["k_wgrad_commit_values", "k_bucket_samples", "k_wgrad_slices"]},
    4: {"check_detectors": ["k_check_detectors_lds"],
        "fill_outputs_fc_i8": ["k_transpose_idx", "k_fill_tm", "k_fill_commit"]},
}


def family_unique_bytes(config):
    """Unique bytes per launch of each family of a configuration (the figures
    the bench line's roofline divides by the family's launch time)."""
    if config == 3:
        B, I, T, Nc, O, _, _ = CONFIGS[3]
        return unique_bytes(B, I, T, Nc, O)
    if config == 4:
        c = INT8
        B, I, T, Nc, O = c["B"], c["I"], c["T"], c["Nc"], c["O"]
        return int8_unique_bytes(B, I, T, Nc, O)
    return {}


def _profile_rows(path):
    import csv
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _timed_rows(rows, warmup, steps):
    """The dispatches of the timed steps: everything from the first dispatch
    of step warmup + 1 on.  A step starts with the first LUT kernel the run
    launches (the earliest dispatch named k_*), which launches the same number
    of times in every step.  Returns (rows, dispatches of that kernel a step,
    its name)."""
    rows = sorted(rows, key=lambda r: (int(r["Start_Timestamp"]), int(r["Dispatch_Id"])))
    marker = next(r["Kernel_Name"] for r in rows if r["Kernel_Name"].startswith("k_"))
    ids = sorted({int(r["Dispatch_Id"]) for r in rows if r["Kernel_Name"] == marker})
    if len(ids) % (warmup + steps):
        raise SystemExit(f"{marker} ran {len(ids)} times, not a multiple of {warmup + steps} steps")
    per_step = len(ids) // (warmup + steps)
    first = ids[warmup * per_step]
    first_ts = min(int(r["Start_Timestamp"]) for r in rows if int(r["Dispatch_Id"]) == first)
    return [r for r in rows if int(r["Start_Timestamp"]) >= first_ts], per_step, marker


def summarize_trace(args):
    """Summary of a rocprofv3 --kernel-trace CSV (run_kernel_trace.csv) over
    the timed steps of a bench.py run: per kernel its launches a step and its
    mean, min and max duration; per launch family the sum of its kernels'
    means; and the dominant family's roofline fraction recomputed from them."""
    import statistics
    rows, per_step, marker = _timed_rows(_profile_rows(args.trace_summary), args.warmup, args.steps)
    by = {}
    for r in rows:
        by.setdefault(r["Kernel_Name"], []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-6)
    total = sum(sum(v) for v in by.values())
    out = [f"# timed steps only: {args.steps} steps after {args.warmup} warm-up steps (from the first "
           f"dispatch of step {args.warmup + 1} of {marker}); times in ms",
           f"{'kernel':<36}{'per_step':>9}{'avg_ms':>10}{'min_ms':>10}{'max_ms':>10}{'ms/step':>10}{'share':>8}"]
    for name, v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"{name[:35]:<36}{len(v) / args.steps:>9.2f}{statistics.fmean(v):>10.4f}{min(v):>10.4f}"
                   f"{max(v):>10.4f}{sum(v) / args.steps:>10.4f}{100 * sum(v) / total:>7.1f}%")
    out.append(f"kernel time per step: {total / args.steps:.4f} ms")
    fams = FAMILIES.get(args.config)
    if fams:
        ub = family_unique_bytes(args.config)
        out.append("")
        out.append("# per launch family: the sum of its kernels' mean durations (bench.py times the family "
                   "with HIP events around the same kernels)")
        fam_ms = {}
        for fam, kernels in fams.items():
            if all(k in by for k in kernels):
                fam_ms[fam] = sum(statistics.fmean(by[k]) for k in kernels)
                out.append(f"{fam:<24}{fam_ms[fam]:>10.4f} ms  = " + " + ".join(kernels))
        if fam_ms:
            dom = max(fam_ms, key=fam_ms.get)
            gbs = ub[dom] / (fam_ms[dom] * 1e-3) / 1e9
            out.append(f"# dominant family {dom}: {ub[dom]} unique bytes / {fam_ms[dom]:.4f} ms = "
                       f"{gbs:.1f} GB/s = {gbs / PEAK_HBM_GBS:.4f} of {PEAK_HBM_GBS:.0f} GB/s")
    print("\n".join(out))


def summarize_counters(args):
    """Summary of rocprofv3 --pmc CSVs (run_counter_collection.csv) over the
    timed steps of a bench.py run: per kernel the mean of each counter per
    dispatch.  FETCH_SIZE and WRITE_SIZE (KiB) become bytes scaled by the
    calibration factors a plain copy of known size gives (--calibration
    FETCH,WRITE); LDS bank-conflict cycles are also given as a fraction of
    the LDS-active cycles.  With --traffic-out, the families' FETCH + WRITE
    bytes per launch (configs 3 and 4) or the whole step's (other configs) go
    to that file, which bench.py reads for roofline.traffic."""
    import statistics
    f_fetch, f_write = (float(v) for v in args.calibration.split(","))
    per = {}
    counters = []
    for path in args.counter_summary:
        rows, per_step, marker = _timed_rows(_profile_rows(path), args.warmup, args.steps)
        for r in rows:
            c = r["Counter_Name"]
            if c not in counters:
                counters.append(c)
            v = float(r["Counter_Value"])
            if c == "FETCH_SIZE":
                v *= 1024 * f_fetch
            elif c == "WRITE_SIZE":
                v *= 1024 * f_write
            per.setdefault(r["Kernel_Name"], {}).setdefault(c, {}).setdefault(r["Dispatch_Id"], 0.0)
            # counters of one dispatch may come as several rows (one per agent block): sum them
            per[r["Kernel_Name"]][c][r["Dispatch_Id"]] += v
    cols = counters + (["conflict_frac"] if {"SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE"} <= set(counters) else [])
    gb = {"FETCH_SIZE", "WRITE_SIZE"}
    out = [f"# timed steps only: {args.steps} steps after {args.warmup} warm-up steps; mean per dispatch; "
           f"FETCH_SIZE / WRITE_SIZE in GB (KiB x 1024 x factor {f_fetch:g} / {f_write:g})",
           f"{'kernel':<30}{'per_step':>9}" + "".join(f"{(c + '_GB' if c in gb else c)[:21]:>22}" for c in cols)]
    means = {}
    order = sorted(per, key=lambda k: -max((statistics.fmean(d.values()) * len(d)
                                            for c, d in per[k].items() if c in ("FETCH_SIZE", "WRITE_SIZE")),
                                           default=0.0))
    for k in order:
        means[k] = {c: statistics.fmean(d.values()) for c, d in per[k].items()}
        n = max(len(d) for d in per[k].values())
        line = f"{k[:29]:<30}{n / args.steps:>9.2f}"
        for c in counters:
            v = means[k].get(c, float("nan"))
            line += f"{v / 1e9:>22.4f}" if c in gb else f"{v:>22.0f}"
        if "conflict_frac" in cols:
            line += f"{means[k]['SQ_LDS_BANK_CONFLICT'] / max(means[k]['SQ_LDS_IDX_ACTIVE'], 1.0):>22.4f}"
        out.append(line)
    print("\n".join(out))
    if args.traffic_out:
        if not {"FETCH_SIZE", "WRITE_SIZE"} <= set(counters):
            raise SystemExit("--traffic-out needs FETCH_SIZE and WRITE_SIZE runs")
        lines = [f"# HBM bytes (FETCH_SIZE + WRITE_SIZE, calibrated) from: " + " ".join(args.counter_summary),
                 f"# sources {source_digest()}"]
        fams = FAMILIES.get(args.config)
        if fams:
            for fam, kernels in fams.items():
                if all(k in means for k in kernels):
                    b = sum(means[k]["FETCH_SIZE"] + means[k]["WRITE_SIZE"] for k in kernels)
                    lines.append(f"{fam} {b:.0f}")
        else:
            step = sum(sum(per[k][c].values()) for k in per for c in ("FETCH_SIZE", "WRITE_SIZE")
                       if c in per[k]) / args.steps
            lines.append(f"step {step:.0f}")
        with open(args.traffic_out, "w") as f:
            f.write("\n".join(lines) + "\n")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the first launches of the config-3 weight gradient run up to 35 % slower
    # (2.24, 2.17, 1.90, 1.81, 1.72, 1.66, 1.63 ms on one MI355X) and settle
    # after about eight steps
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=3, choices=sorted(CONFIGS) + [2, 4, 5])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--product", action="store_true",
                    help="time the product-mode LUT layer (concatenation_product=False) instead")
    ap.add_argument("--densify", action="store_true",
                    help="time the dense -> sparse gradient converter instead of a LUT config")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="only run a plain copy of this many MiB (counter calibration) and exit")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarise a rocprofv3 kernel trace of a bench.py run with the same --config, "
                         "--steps and --warmup over its timed steps, and exit")
    ap.add_argument("--counter-summary", metavar="CSV", nargs="+",
                    help="summarise rocprofv3 --pmc CSVs of a bench.py run with the same --config, "
                         "--steps and --warmup over its timed steps, and exit")
    ap.add_argument("--calibration", default="2,1",
                    help="FETCH_SIZE,WRITE_SIZE scale factors from a copy of known size")
    ap.add_argument("--traffic-out", metavar="FILE",
                    help="with --counter-summary: write the HBM bytes per family (or per step) here")
    args = ap.parse_args()
    if args.calibrate_copy_mib:
        calibrate_copy(args.calibrate_copy_mib)
        return
    if args.trace_summary:
        summarize_trace(args)
        return
    if args.counter_summary:
        summarize_counters(args)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build's LUT path runs on a single MI355X "
              "(the multi-GPU table-parallel design is described, not built).", file=sys.stderr)
        sys.exit(2)

    if args.product:
        return bench_product(args)
    if args.densify:
        bench_densify(args)
        return
    if args.config == 5:
        bench_transformer(args)
        return
    if args.config == 4:
        bench_int8(args)
        return
    if args.config == 2:
        bench_projection(args)
        return

    import torch
    from spiky_amd import LUTLayer

    B, I, T, Nc, O, xdist, cpu_B = CONFIGS[args.config]
    E = 1 << Nc
    dev = torch.device("cuda:0")
    log(f"config {args.config}: B={B} I={I} T={T} Nc={Nc} O={O}")
    anchors = make_anchors(T, I, Nc, 1, dev)
    layer = LUTLayer(I, Nc, T, O, _explicit_anchors=anchors, device=dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    with torch.no_grad():
        layer._weights.normal_(0.0, 0.01, generator=gen)
    gx = torch.Generator(device=dev).manual_seed(0)
    x = (torch.randn(B, 1, I, device=dev, generator=gx) if xdist == "normal"
         else torch.rand(B, 1, I, device=dev, generator=gx))
    x.requires_grad_(True)
    gg = torch.Generator(device=dev).manual_seed(3)
    go = torch.randn(B, 1, O, device=dev, generator=gg)
    dm = layer._lut_dm

    def step():
        layer._weights.grad = None
        x.grad = None
        y = layer(x)
        y.backward(go)

    log("warmup")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    dm.get_kernel_times(reset=True)
    dm.set_kernel_timing(True)
    log(f"timing {args.steps} steps")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    dm.set_kernel_timing(False)
    ktimes = dm.get_kernel_times(reset=True)
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    value = B / (ms_per_step / 1e3)
    log(f"{ms_per_step:.3f} ms/step, {value:.1f} samples/s; kernels {ktimes}")

    gbytes = g_model_bytes(B, I, T, Nc, O)
    ubytes = unique_bytes(B, I, T, Nc, O)
    per_kernel = {}
    for name, (cnt, tot) in ktimes.items():
        ms = tot / max(cnt, 1)
        per_kernel[name] = {"ms_per_launch": round(ms, 4),
                            "unique_gbs": round(ubytes[name] / (ms * 1e-3) / 1e9, 1) if name in ubytes else None,
                            "g_model_gbs": round(gbytes[name] / (ms * 1e-3) / 1e9, 1) if name in gbytes else None}
    dom = max(ktimes.items(), key=lambda kv: kv[1][1])[0]
    dom_ms = ktimes[dom][1] / ktimes[dom][0]
    achieved = ubytes[dom] / (dom_ms * 1e-3) / 1e9
    traffic, digest = load_traffic(dom, args.config)
    stale = traffic is not None and digest != source_digest()
    if stale:
        traffic = None
    step_g = sum(gbytes.values())
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        # unique bytes of one launch (each tensor once) over its mean launch time
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "algorithmic_bytes_per_launch": ubytes[dom],
        "ms_per_launch": round(dom_ms, 4),
        # measured HBM bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE,
        # profiles/hbm_traffic_config3.txt), null when that summary predates
        # the current kernel sources
        "traffic": traffic,
        "traffic_source_digest": digest,
        "traffic_stale": stale,
        "traffic_gbs": round(traffic / (dom_ms * 1e-3) / 1e9, 1) if traffic else None,
        "traffic_frac": round(traffic / (dom_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4) if traffic else None,
        # the gather model (every sample's row access counted, no reuse credit):
        # above 1 wherever the table-major kernels serve rows from LDS
        "g_model": {"bytes_per_launch": gbytes[dom],
                    "frac": round(gbytes[dom] / (dom_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                    "step_frac": round(step_g / (ms_per_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        "step_compulsory_frac": round(compulsory_bytes(B, I, T, Nc, O) / (ms_per_step * 1e-3) / 1e9
                                      / PEAK_HBM_GBS, 4),
        "kernels": per_kernel,
    }
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(x.detach().reshape(-1), layer._detector_anchors, layer._weights.detach(),
                           go.reshape(-1), B, I, T, Nc, O, cpu_B)
    res = {
        "metric": "LUT fwd+bwd samples/sec at 8192 tables; achieved HBM GB/s vs peak",
        "value": round(value, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (fp64 partial sums)",
        "data": "synthetic (seeded N(0,1) inputs and grads, N(0,0.01) tables, anchors without replacement)",
        "config": {"workload": f"BASELINE config {args.config}: dense LUT layer fwd+bwd", "batch": B,
                   "n_inputs": I, "n_tables": T, "anchors_per_table": Nc, "n_outputs": O,
                   "table_bytes": T * E * O * 4, "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
