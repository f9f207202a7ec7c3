// lut_sparse.hip -- sparse (ProjectionLUTLayer) LUT kernels for gfx950.
//
// Connectivity is this build's CSR (see lut_kernels.h): lookup neuron
// n = t*E + e owns synapses [syn_offsets[n], syn_offsets[n+1]) with output
// indices syn_targets[s] and one fp32 weight w[s] each.  A neuron's synapses
// form forward groups of `ogs` (forward_group_size) in list order, the unit of
// the reference's ForwardSynapseGroup (connections_manager.h:39-66).
//
//   k_fill_sparse_uniform  one thread per (b, output): walks the outputs'
//                          incoming (detector, slot) pairs in ascending order,
//                          which is the reference CPU path's commit order, so the
//                          fp32 result is bit-identical to it (no atomics).
//   k_keys_by_table        the lookup indices table-major, one byte (or two) a
//                          key: keys_t[t][b] = idx[b][t].
//   k_fill_sparse_by_sample the same sums with a wavefront per (output, 64
//                          samples), outputs longest list first: the list is
//                          read through scalar loads once per 64 samples and the
//                          keys of 64 samples are 64 contiguous bytes.
//   k_fill_sparse_atomic   one thread per (b, t, group): the reference's own
//                          decomposition with fp32/int32 atomics (any topology).
//   k_propagate_sparse     eight lanes (one for int32 sums) per (b, t, group):
//                          main/alt group dots in fp64 and the min-margin anchor
//                          update.
//   k_propagate_sparse_rows the same for fp32 sums over uniform rows: four lanes
//                          per (b, t, group), each with a fixed number of entry
//                          slots, the row's targets read once for both rows,
//                          three rounds of loads, none behind a branch, and the
//                          input-gradient adds summed in LDS where inputs are few.
//   k_wgrad_sparse_rowsum  one thread per synapse: sums lr*g over the samples
//                          bucketed on its lookup neuron (read from a per-synapse
//                          neuron index), ascending (bit-identical to the
//                          reference CPU path), and writes it once.
//   k_wgrad_sparse_cols    the same sums over uniform rows, one thread per
//                          (table, synapse slot, four rows): one sample walk
//                          serves the four rows' synapses of one target.
#include "lut_kernels.h"

#include <algorithm>

namespace spiky {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

__device__ __forceinline__ double du_of_margin(float md) {
    double du = (double)md;
    double r = 1.0 / (1.0 + fabs(du));
    return (du > 0) ? r * (0.5 * r) : r * (-0.5 * r);
}

uint32_t blocks_for(uint64_t n) { return (uint32_t)((n + kBlock - 1) / kBlock); }

// fill_outputs_non_seq_sparse_logic (lut_runtime_kernels_logic.proto:1160-1212)
// with fire_single_synapse_group (proto:215-313): every synapse commits
// (float)(double)w, or the int32 payload trunc(w*DENOM32*int_rescaler).
template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_fill_sparse_uniform(
    const float *__restrict__ w, const int32_t *__restrict__ idx,
    const int64_t *__restrict__ syn_offsets, const int64_t *__restrict__ in_offsets,
    const int4 *__restrict__ in_pairs, float *__restrict__ out, uint32_t batch,
    uint32_t n_outputs, uint32_t n_detectors, uint32_t n_entries, double int_rescaler) {
    const uint64_t item = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (item >= (uint64_t)batch * n_outputs) return;
    const uint32_t b = (uint32_t)(item / n_outputs);
    const uint32_t j = (uint32_t)(item % n_outputs);
    const int32_t *ib = idx + (size_t)b * n_detectors;
    float acc = out[item];
    int32_t iacc = __float_as_int(acc);
    const uint32_t emask = n_entries - 1;
    // unrolled so that several pairs' dependent loads (entry, index, weight)
    // are in flight at once; the adds stay in ascending pair order.  An entry
    // holds the synapse's offset in the detector's row 0 and the row length,
    // so the weight's address needs no neuron offset load.
#pragma unroll 8
    for (int64_t p = in_offsets[j]; p < in_offsets[j + 1]; p++) {
        const int4 tk = in_pairs[p];
        const uint32_t e = (uint32_t)ib[tk.x] & emask;
        const double wt = (double)w[(uint32_t)tk.y + e * (uint32_t)tk.z];
        if (INT_MODE)
            iacc = wrap_add(iacc, (int32_t)(wt * kDenom32 * int_rescaler));
        else
            acc += (float)wt;
    }
    if (INT_MODE)
        out[item] = (float)(((double)iacc * kDenom32Reciproc) / int_rescaler);
    else
        out[item] = acc;
}

// Thread (t4, b): keys_t[t][b] = idx[b][t] for t = 4 t4 .. 4 t4 + 3, lanes
// running over b (the 16-byte reads when rows are 16-byte aligned, `vec`).
template <typename KT>
__global__ __launch_bounds__(kBlock) void k_keys_by_table(const int32_t *__restrict__ idx, KT *__restrict__ keys_t,
                                                          uint32_t batch, uint32_t n_detectors, bool vec) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    const uint32_t n_t4 = (n_detectors + 3) / 4;
    if (i >= (uint64_t)n_t4 * batch) return;
    const uint32_t b = (uint32_t)(i % batch), t = (uint32_t)(i / batch) * 4;
    const int32_t *src = idx + (size_t)b * n_detectors + t;
    KT *dst = keys_t + (size_t)t * batch + b;
    if (vec) {
        const int4 v = *reinterpret_cast<const int4 *>(src);
        dst[0] = (KT)v.x;
        dst[batch] = (KT)v.y;
        dst[2 * (size_t)batch] = (KT)v.z;
        dst[3 * (size_t)batch] = (KT)v.w;
    } else {
        for (uint32_t k = 0; k < 4 && t + k < n_detectors; k++) dst[k * (size_t)batch] = (KT)src[k];
    }
}

// The sums of k_fill_sparse_uniform, one wavefront (a workgroup) per (output
// order[r], 64 samples), lane = sample.  The output's list is the same for
// every lane, so it comes through scalar loads, and lane b's key of table t is
// keys_t[t * batch + b]: 64 lanes read 64 (or 128) contiguous bytes.  The walk
// runs three groups of kGrp entries deep -- the weights of group g, the keys of
// group g + 1 and the entries of group g + 2 are in flight together -- and adds
// in ascending entry order, so the result is bit-identical to the one-thread
// walk.  Outputs come longest list first (order[]), so the longest walks start
// first and the short ones fill in behind them.
constexpr int kSparseGrp = 8;
constexpr uint32_t kSparseLanesMinBatch = 48;

template <bool INT_MODE, typename KT>
__global__ __launch_bounds__(64) void k_fill_sparse_by_sample(
    const float *__restrict__ w, const KT *__restrict__ keys_t, const int64_t *__restrict__ in_offsets,
    const int4 *__restrict__ in_pairs, const uint32_t *__restrict__ order, float *__restrict__ out,
    uint32_t batch, uint32_t n_outputs, uint32_t n_bblk, uint32_t emask, double int_rescaler) {
    constexpr int G = kSparseGrp;
    const uint32_t r = blockIdx.x / n_bblk;
    const uint32_t j = __builtin_amdgcn_readfirstlane(order[r]);
    const uint32_t b = (blockIdx.x % n_bblk) * 64u + threadIdx.x;
    const bool on = b < batch;
    const uint32_t bb = on ? b : batch - 1u;  // lanes past the batch walk a valid sample
    const size_t o = (size_t)bb * n_outputs + j;
    const KT *kb = keys_t + bb;
    float acc = out[o];
    int32_t iacc = __float_as_int(acc);
    const int64_t p0 = in_offsets[j], p1 = in_offsets[j + 1];
    const int64_t ng = (p1 - p0) / G;
    int4 pa[G], pb[G];
    uint32_t ea[G];
#pragma unroll
    for (int k = 0; k < G; k++) {
        pa[k] = make_int4(0, 0, 0, 0);
        pb[k] = pa[k];
        ea[k] = 0;
    }
    if (ng > 0) {
        const int64_t pn = ng > 1 ? p0 + G : p0;
#pragma unroll
        for (int k = 0; k < G; k++) {
            pa[k] = in_pairs[p0 + k];
            pb[k] = in_pairs[pn + k];
        }
#pragma unroll
        for (int k = 0; k < G; k++) ea[k] = kb[(size_t)pa[k].x * batch];
    }
    // The values entering the loop pass through an xor with a zero the
    // compiler cannot prove, so no loop-carried value is a phi of loads alone:
    // the optimiser would turn such a phi into one load at the use, which
    // undoes the three-deep walk.
    const uint32_t z = emask >> 31;
#pragma unroll
    for (int k = 0; k < G; k++) {
        pa[k].x ^= z; pa[k].y ^= z; pa[k].z ^= z;
        pb[k].x ^= z; pb[k].y ^= z; pb[k].z ^= z;
        ea[k] ^= z;
    }
    // past the last group the entry loads re-read group 0 (in bounds, unused):
    // the loop has no branch, so its waits count the loads in flight exactly
    for (int64_t g = 0; g < ng; g++) {
        float wv[G];
        uint32_t eb[G];
        int4 pc[G];
#pragma unroll
        for (int k = 0; k < G; k++) wv[k] = w[(uint32_t)pa[k].y + (ea[k] & emask) * (uint32_t)pa[k].z];
#pragma unroll
        for (int k = 0; k < G; k++) eb[k] = kb[(size_t)pb[k].x * batch];
        const int64_t pn = (g + 2 < ng) ? p0 + (g + 2) * G : p0;
#pragma unroll
        for (int k = 0; k < G; k++) pc[k] = in_pairs[pn + k];
#pragma unroll
        for (int k = 0; k < G; k++) {
            const double wt = (double)wv[k];
            if (INT_MODE)
                iacc = wrap_add(iacc, (int32_t)(wt * kDenom32 * int_rescaler));
            else
                acc += (float)wt;
        }
#pragma unroll
        for (int k = 0; k < G; k++) {
            pa[k] = pb[k];
            ea[k] = eb[k];
            pb[k] = pc[k];
        }
    }
#pragma unroll 8
    for (int64_t p = p0 + ng * G; p < p1; p++) {
        const int4 tk = in_pairs[p];
        const uint32_t e = (uint32_t)kb[(size_t)tk.x * batch] & emask;
        const double wt = (double)w[(uint32_t)tk.y + e * (uint32_t)tk.z];
        if (INT_MODE)
            iacc = wrap_add(iacc, (int32_t)(wt * kDenom32 * int_rescaler));
        else
            acc += (float)wt;
    }
    if (!on) return;
    if (INT_MODE)
        out[o] = (float)(((double)iacc * kDenom32Reciproc) / int_rescaler);
    else
        out[o] = acc;
}

template <typename KT>
hipError_t launch_fill_by_sample(const SparseShape &s, const float *w, const int32_t *idx,
                                 const int64_t *in_offsets, const int4 *pairs, const uint32_t *order,
                                 uint32_t n_order, float *out, bool int_mode, double int_rescaler, Scratch &scr,
                                 hipStream_t st) {
    ScratchLayout lay(scr);
    KT *keys_t = lay.take<KT>((size_t)s.fc.n_detectors * s.fc.batch * sizeof(KT));
    hipError_t e;
    if (lay.stop(&e, "fill_outputs_sparse")) return e;
    const uint64_t n_keys = (uint64_t)((s.fc.n_detectors + 3) / 4) * s.fc.batch;
    const uint32_t n_bblk = (s.fc.batch + 63) / 64;
    const uint64_t grid = (uint64_t)n_order * n_bblk;
    if (grid > 0x7fffffffu || (n_keys + kBlock - 1) / kBlock > 0x7fffffffu) return hipErrorInvalidConfiguration;
    if (grid == 0) return hipSuccess;
    const bool vec = s.fc.n_detectors % 4 == 0 && reinterpret_cast<uintptr_t>(idx) % 16 == 0;
    hipLaunchKernelGGL(k_keys_by_table<KT>, dim3((uint32_t)((n_keys + kBlock - 1) / kBlock)), dim3(kBlock), 0, st,
                       idx, keys_t, s.fc.batch, s.fc.n_detectors, vec);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t emask = s.fc.n_entries - 1;
    if (int_mode)
        hipLaunchKernelGGL((k_fill_sparse_by_sample<true, KT>), dim3((uint32_t)grid), dim3(64), 0, st, w, keys_t,
                           in_offsets, pairs, order, out, s.fc.batch, s.fc.n_outputs, n_bblk, emask, int_rescaler);
    else
        hipLaunchKernelGGL((k_fill_sparse_by_sample<false, KT>), dim3((uint32_t)grid), dim3(64), 0, st, w, keys_t,
                           in_offsets, pairs, order, out, s.fc.batch, s.fc.n_outputs, n_bblk, emask, int_rescaler);
    return hipGetLastError();
}

template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_fill_sparse_atomic(
    const float *__restrict__ w, const int32_t *__restrict__ idx,
    const int64_t *__restrict__ syn_offsets, const int32_t *__restrict__ syn_targets,
    float *__restrict__ out, uint32_t n_outputs, uint32_t n_detectors, uint32_t n_entries,
    uint32_t ogs, uint32_t max_groups, uint64_t n_items, double int_rescaler) {
    const uint64_t item = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (item >= n_items) return;
    const uint32_t grp = (uint32_t)(item % max_groups);
    const uint64_t bt = item / max_groups;
    const uint32_t t = (uint32_t)(bt % n_detectors);
    const uint32_t b = (uint32_t)(bt / n_detectors);
    const uint32_t n = t * n_entries + ((uint32_t)idx[bt] & (n_entries - 1));
    const int64_t s0 = syn_offsets[n] + (int64_t)grp * ogs;
    const int64_t s1 = min(s0 + (int64_t)ogs, syn_offsets[n + 1]);
    float *ob = out + (size_t)b * n_outputs;
    for (int64_t s = s0; s < s1; s++) {
        const uint32_t tg = (uint32_t)syn_targets[s];
        if (tg >= n_outputs) continue;
        const double wt = (double)w[s];
        if (INT_MODE)
            atomicAdd(reinterpret_cast<int32_t *>(ob + tg), (int32_t)(wt * kDenom32 * int_rescaler));
        else
            unsafeAtomicAdd(ob + tg, (float)wt);
    }
}

// propagate_through_detectors_non_seq_sparse_logic (proto:1303-1419) with
// accumulate_grad_sum_sparse (proto:315-395).  fp32 summation: eight lanes per
// (b, t, group): lane l takes the group's synapses l, l + 8, .. of the main and
// of the alternative neuron (fp64 sums of the exact products w * g), the eight
// partial sums are joined by DPP (a tree of depth 3), and lane 0 applies the
// min-margin anchor update; the eight lanes of an item share its early exits.
// int32 summation keeps one lane per item and the synapses' serial order, so
// the fp64 dot, and with it the truncated payload, is the reference's.
template <bool INT_MODE>
constexpr int sp_lanes() { return INT_MODE ? 1 : 8; }

__device__ __forceinline__ double sp_dpp_f64(double v, int ctrl_sel) {
    const long long u = __double_as_longlong(v);
    int lo = (int)(uint32_t)u, hi = (int)(uint32_t)((unsigned long long)u >> 32);
    if (ctrl_sel == 0) {
        lo = __builtin_amdgcn_mov_dpp(lo, 0xB1, 0xF, 0xF, true);  // quad_perm xor 1
        hi = __builtin_amdgcn_mov_dpp(hi, 0xB1, 0xF, 0xF, true);
    } else if (ctrl_sel == 1) {
        lo = __builtin_amdgcn_mov_dpp(lo, 0x4E, 0xF, 0xF, true);  // quad_perm xor 2
        hi = __builtin_amdgcn_mov_dpp(hi, 0x4E, 0xF, 0xF, true);
    } else {
        lo = __builtin_amdgcn_mov_dpp(lo, 0x141, 0xF, 0xF, true);  // half-row mirror (8 lanes)
        hi = __builtin_amdgcn_mov_dpp(hi, 0x141, 0xF, 0xF, true);
    }
    return __longlong_as_double((long long)(((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo));
}

// sum over the 8 lanes of a group, every lane gets it
__device__ __forceinline__ double sp_sum4(double v) {
    v += sp_dpp_f64(v, 0);
    v += sp_dpp_f64(v, 1);
    return v;
}

__device__ __forceinline__ double sp_sum8(double v) {
    v += sp_dpp_f64(v, 0);
    v += sp_dpp_f64(v, 1);
    v += sp_dpp_f64(v, 2);
    return v;
}

template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_propagate_sparse(
    const float *__restrict__ w, const float *__restrict__ g, const int32_t *__restrict__ idx,
    const float *__restrict__ md, const int32_t *__restrict__ mi, const int2 *__restrict__ anchors,
    const int64_t *__restrict__ syn_offsets, const int32_t *__restrict__ syn_targets,
    float *__restrict__ x_grad, uint32_t n_inputs, uint32_t n_outputs, uint32_t n_detectors,
    uint32_t n_anchors, uint32_t n_entries, uint32_t ogs, uint32_t max_groups, uint64_t n_items,
    double int_rescaler, bool uniform) {
    constexpr int kSpLanes = sp_lanes<INT_MODE>();
    const uint64_t gid = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    const uint64_t item = gid / kSpLanes;
    const uint32_t l = (uint32_t)(gid % kSpLanes);
    if (item >= n_items) return;  // whole lane groups (kBlock % 8 == 0)
    const uint32_t grp = (uint32_t)(item % max_groups);
    const uint64_t bt = item / max_groups;
    const uint32_t t = (uint32_t)(bt % n_detectors);
    const uint32_t b = (uint32_t)(bt / n_detectors);
    // uniform rows: row e of detector t starts at o0 + e * len, read beside the
    // index instead of after it
    const int64_t o0 = uniform ? syn_offsets[(size_t)t * n_entries] : 0;
    const int64_t len = uniform ? syn_offsets[(size_t)t * n_entries + 1] - o0 : 0;
    const int32_t m = mi[bt];
    if (m < 0 || (uint32_t)m >= n_anchors) return;
    const uint32_t r = (uint32_t)idx[bt] & (n_entries - 1);
    const uint32_t nm = t * n_entries + r;
    const uint32_t na = t * n_entries + (r ^ (1u << m));
    const int64_t bm = uniform ? o0 + (int64_t)r * len : syn_offsets[nm];
    const int64_t em = uniform ? bm + len : syn_offsets[nm + 1];
    const int64_t ba = uniform ? o0 + (int64_t)(r ^ (1u << m)) * len : syn_offsets[na];
    const int64_t ea = uniform ? ba + len : syn_offsets[na + 1];
    const float *gb = g + (size_t)b * n_outputs;
    double ms = 0.0, as = 0.0;
    {
        const int64_t s0 = bm + (int64_t)grp * ogs;
        const int64_t s1 = min(s0 + (int64_t)ogs, em);
        for (int64_t s = s0 + l; s < s1; s += kSpLanes) {
            const uint32_t tg = (uint32_t)syn_targets[s];
            if (tg < n_outputs) ms += (double)w[s] * (double)gb[tg];
        }
    }
    {
        const int64_t s0 = ba + (int64_t)grp * ogs;
        const int64_t s1 = min(s0 + (int64_t)ogs, ea);
        for (int64_t s = s0 + l; s < s1; s += kSpLanes) {
            const uint32_t tg = (uint32_t)syn_targets[s];
            if (tg < n_outputs) as += (double)w[s] * (double)gb[tg];
        }
    }
    if (kSpLanes == 8) {
        ms = sp_sum8(ms);
        as = sp_sum8(as);
        if (l != 0) return;
    }
    const double du = du_of_margin(md[bt]) * (ms - as);
    if (!(fabs(du) > kEps)) return;
    const int2 a = anchors[(size_t)t * n_anchors + m];
    if ((uint32_t)a.x >= n_inputs || (uint32_t)a.y >= n_inputs) return;
    float *xg = x_grad + (size_t)b * n_inputs;
    if (INT_MODE) {
        const int32_t d = (int32_t)(du * kDenom32 * int_rescaler);
        atomicAdd(reinterpret_cast<int32_t *>(xg + a.x), d);
        atomicAdd(reinterpret_cast<int32_t *>(xg + a.y), (int32_t)(0u - (uint32_t)d));
    } else {
        unsafeAtomicAdd(xg + a.x, (float)du);
        unsafeAtomicAdd(xg + a.y, (float)(-du));
    }
}

// k_propagate_sparse for fp32 sums when every lookup neuron of a detector has
// the same target list: kRowLanes lanes per (b, t, group), P entry slots a
// lane per pass over the group, grid (items, batch).  The rows of a detector
// share their targets, so the main and the alternative row read one target
// and one output gradient per entry.  The loads go out in three rounds --
// (offsets, key, min-margin index), then (margin, anchors, targets, both
// rows' weights), then the output gradients -- with no branch between them
// for groups of at most P * kRowLanes entries; slots past the group read
// synapse 0 (in bounds) and add nothing.  With RED the workgroup (one sample)
// first sums its input-gradient adds in LDS and then adds each non-zero input
// once: where many tables share few inputs, that takes most of the same-address
// atomics off the L2.
constexpr int kRowLanes = 4;
constexpr uint32_t kRowRedInputs = 4096;  // the LDS sum's inputs (16 KiB)

template <int P, bool RED>
__global__ __launch_bounds__(kBlock) void k_propagate_sparse_rows(
    const float *__restrict__ w, const float *__restrict__ g, const int32_t *__restrict__ idx,
    const float *__restrict__ md, const int32_t *__restrict__ mi, const int2 *__restrict__ anchors,
    const int64_t *__restrict__ syn_offsets, const int32_t *__restrict__ syn_targets,
    float *__restrict__ x_grad, uint32_t n_inputs, uint32_t n_outputs, uint32_t n_detectors,
    uint32_t n_anchors, uint32_t n_entries, uint32_t ogs, uint32_t max_groups, uint32_t n_items) {
    constexpr int L = kRowLanes;
    __shared__ float red[RED ? kRowRedInputs : 1];
    if (RED) {
        for (uint32_t i = threadIdx.x; i < n_inputs; i += kBlock) red[i] = 0.0f;
        __syncthreads();
    }
    const uint32_t xi = blockIdx.x * kBlock + threadIdx.x;
    const uint32_t l = xi % L;
    const uint32_t item0 = xi / L;  // t * max_groups + group
    if (!RED && item0 >= n_items) return;  // whole lane groups (kBlock % L == 0)
    const bool live = item0 < n_items;
    const uint32_t item = live ? item0 : 0u;  // past the end: item 0's loads, no adds
    const uint32_t b = blockIdx.y;
    const uint32_t grp = max_groups == 1 ? 0 : item % max_groups;
    const uint32_t t = max_groups == 1 ? item : item / max_groups;
    const size_t bt = (size_t)b * n_detectors + t;
    const int64_t o0 = syn_offsets[(size_t)t * n_entries];
    const int64_t o1 = syn_offsets[(size_t)t * n_entries + 1];
    const int32_t m = mi[bt];
    const uint32_t r = (uint32_t)idx[bt] & (n_entries - 1);
    const float mdv = md[bt];
    // the 64-bit length keeps both halves of the offsets' load live, so no
    // register of it is reused (and waited for) before the other loads go out
    const int64_t len64 = o1 - o0;
    const uint32_t len = (uint32_t)len64;
    const uint32_t k0 = grp * ogs;
    const uint32_t k1 = min(k0 + ogs, len);
    const bool act = m >= 0 && (uint32_t)m < n_anchors;
    const uint32_t mm = act ? (uint32_t)m : 0u;
    const int2 a = anchors[(size_t)t * n_anchors + mm];
    const int64_t om = o0 + (int64_t)r * len64, oa = o0 + (int64_t)(r ^ (1u << mm)) * len64;
    const float *gb = g + (size_t)b * n_outputs;
    double ms = 0.0, as = 0.0;
    for (uint32_t c0 = k0; c0 < k1; c0 += (uint32_t)(L * P)) {
        uint32_t tgv[P];
        float wmv[P], wav[P];
        bool ok[P];
#pragma unroll
        for (int i = 0; i < P; i++) {
            const uint32_t k = c0 + l + (uint32_t)i * L;
            ok[i] = k < k1;
            tgv[i] = (uint32_t)syn_targets[ok[i] ? o0 + k : 0];
            wmv[i] = w[ok[i] ? om + k : 0];
            wav[i] = w[ok[i] ? oa + k : 0];
        }
        double gv[P];
#pragma unroll
        for (int i = 0; i < P; i++) gv[i] = (double)gb[tgv[i]];
#pragma unroll
        for (int i = 0; i < P; i++) {
            const double pm = ms + (double)wmv[i] * gv[i], pa = as + (double)wav[i] * gv[i];
            ms = ok[i] ? pm : ms;
            as = ok[i] ? pa : as;
        }
    }
    // The margin and the anchors are used in this block, so their loads stay up
    // front instead of sinking below a branch; dmg == 0 gives du == 0, which
    // never fires, so testing it changes nothing.
    const double dmg = du_of_margin(mdv);
    const bool fire = live && act && (uint32_t)a.x < n_inputs && (uint32_t)a.y < n_inputs && dmg != 0.0;
    ms = sp_sum4(ms);
    as = sp_sum4(as);
    const double du = dmg * (ms - as);
    const bool add = l == 0 && fire && fabs(du) > kEps;
    float *xg = x_grad + (size_t)b * n_inputs;
    if (RED) {
        if (add) {
            atomicAdd(&red[a.x], (float)du);
            atomicAdd(&red[a.y], (float)(-du));
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < n_inputs; i += kBlock) {
            const float v = red[i];
            if (v != 0.0f) unsafeAtomicAdd(xg + i, v);
        }
    } else if (add) {
        unsafeAtomicAdd(xg + a.x, (float)du);
        unsafeAtomicAdd(xg + a.y, (float)(-du));
    }
}

// gather_w_gradients_non_seq_sparse_logic (proto:1501-1545) with
// gather_weight_gradients_sparse (proto:584-714), one thread per synapse.
// The neuron of synapse s is syn_neuron[s].  With OVERWRITE the target starts
// from zero and is not read (the caller need not clear it).
template <bool INT_MODE, bool OVERWRITE>
__global__ __launch_bounds__(kBlock) void k_wgrad_sparse_rowsum(
    const float *__restrict__ g, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ samples, const int32_t *__restrict__ syn_neuron,
    const int32_t *__restrict__ syn_targets, float *__restrict__ target, uint32_t batch,
    uint32_t n_outputs, uint32_t n_entries, uint64_t n_synapses, double lr, double int_rescaler) {
    const uint64_t s = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (s >= n_synapses) return;
    const uint32_t n = (uint32_t)syn_neuron[s];
    const uint32_t t = n / n_entries;
    const uint32_t e = n % n_entries;
    const int32_t *off_t = offsets + (size_t)t * (n_entries + 1);
    const int32_t beg = off_t[e], end = off_t[e + 1];
    const uint32_t tg = (uint32_t)syn_targets[s];
    const float init = OVERWRITE ? 0.0f : target[s];
    if (beg == end || tg >= n_outputs) {
        if (INT_MODE) {
            const double y = (double)__float_as_int(init) * kDenom32Reciproc;
            target[s] = (float)(y / int_rescaler);
        } else if (OVERWRITE) {
            target[s] = 0.0f;
        }
        return;
    }
    const int32_t *smp = samples + (size_t)t * batch;
    float acc = init;
    int32_t iacc = __float_as_int(acc);
    // unrolled: several samples' g loads in flight, the adds in ascending order
#pragma unroll 4
    for (int32_t k = beg; k < end; k++) {
        const double gg = (double)g[(size_t)smp[k] * n_outputs + tg];
        if (!(fabs(gg) > kEps)) continue;
        if (INT_MODE)
            iacc = wrap_add(iacc, (int32_t)(gg * lr * kDenom32 * int_rescaler));
        else
            acc += (float)(gg * lr);
    }
    if (INT_MODE)
        target[s] = (float)(((double)iacc * kDenom32Reciproc) / int_rescaler);
    else
        target[s] = acc;
}

// k_wgrad_sparse_rowsum over uniform rows, one thread per (t, k, row chunk):
// synapse k of rows [e0, e1) of detector t (the rows share its target),
// walking those rows' samples in bucket order -- row by row, each row's samples
// ascending -- and closing row e when its bucket ends.  Lanes of one (t, row
// chunk) walk one sample list; the output-gradient loads of kWgChunk samples go
// out together with the next chunk's sample ids, and the adds stay in
// ascending order within each row (bit-identical to the per-synapse walk).  A
// row's start value and the next bucket's end are loaded one row ahead.
constexpr int kWgChunk = 16;

template <bool INT_MODE, bool OVERWRITE>
__global__ __launch_bounds__(kBlock) void k_wgrad_sparse_cols(
    const float *__restrict__ g, const int32_t *__restrict__ offsets, const int32_t *__restrict__ samples,
    const int2 *__restrict__ pairs, const int64_t *__restrict__ syn_offsets,
    const int32_t *__restrict__ syn_targets, float *__restrict__ target, uint32_t batch, uint32_t n_outputs,
    uint32_t n_entries, uint32_t n_pairs, uint32_t rows_per_chunk, uint64_t n_threads, double lr,
    double int_rescaler) {
    constexpr int C = kWgChunk;
    const uint64_t gid = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (gid >= n_threads) return;
    const uint32_t i = (uint32_t)(gid % n_pairs);
    const uint32_t e0 = (uint32_t)(gid / n_pairs) * rows_per_chunk;
    const uint32_t e1 = min(e0 + rows_per_chunk, n_entries);
    const int2 tk = pairs[i];
    const uint32_t t = (uint32_t)tk.x, k = (uint32_t)tk.y;
    const int64_t o0 = syn_offsets[(size_t)t * n_entries];
    const int64_t len = syn_offsets[(size_t)t * n_entries + 1] - o0;
    const uint32_t tg = (uint32_t)syn_targets[o0 + k];
    const int32_t *off_t = offsets + (size_t)t * (n_entries + 1);
    const int32_t *smp = samples + (size_t)t * batch;
    const float *gc = g + tg;
    float *col = target + o0 + k;  // row e's synapse k at col[e * len]
    const int32_t jb = off_t[e0], je = off_t[e1];
    uint32_t e = e0;
    int32_t end = off_t[e0 + 1];
    int32_t end2 = e0 + 1 < e1 ? off_t[e0 + 2] : je;
    float nxt = (!OVERWRITE && e0 + 1 < e1) ? col[(size_t)(e0 + 1) * len] : 0.0f;
    float acc = OVERWRITE ? 0.0f : col[(size_t)e0 * len];
    int32_t iacc = __float_as_int(acc);
    auto close_row = [&]() {
        col[(size_t)e * len] = INT_MODE ? (float)(((double)iacc * kDenom32Reciproc) / int_rescaler) : acc;
    };
    auto next_row = [&]() {
        close_row();
        e++;
        acc = nxt;
        iacc = __float_as_int(nxt);
        end = end2;
        if (e + 1 < e1) {
            end2 = off_t[e + 2];
            if (!OVERWRITE) nxt = col[(size_t)(e + 1) * len];
        }
    };
    const int32_t jl = max(je - 1, 0);  // a valid position for the loads past the range
    int32_t sv[C];
#pragma unroll
    for (int c = 0; c < C; c++) sv[c] = smp[min(jb + c, jl)];
    // the sample ids entering the loop pass through an xor with a zero the
    // compiler cannot prove, so they are not folded into loads at the use
    const int32_t z = (int32_t)(n_entries >> 31);
#pragma unroll
    for (int c = 0; c < C; c++) sv[c] ^= z;
    for (int32_t j0 = jb; j0 < je; j0 += C) {
        float gv[C];
        int32_t sn[C];
#pragma unroll
        for (int c = 0; c < C; c++) gv[c] = gc[(size_t)(uint32_t)sv[c] * n_outputs];
#pragma unroll
        for (int c = 0; c < C; c++) sn[c] = smp[min(j0 + C + c, jl)];
#pragma unroll
        for (int c = 0; c < C; c++) {
            const int32_t j = j0 + c;
            if (j < je) {
                while (j == end) next_row();
                const double gg = (double)gv[c];
                if (fabs(gg) > kEps) {
                    if (INT_MODE)
                        iacc = wrap_add(iacc, (int32_t)(gg * lr * kDenom32 * int_rescaler));
                    else
                        acc += (float)(gg * lr);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < C; c++) sv[c] = sn[c];
    }
    // the last sample's row, then every row of the chunk after it (empty buckets)
    while (e + 1 < e1) next_row();
    close_row();
}

}  // namespace

bool sparse_fill_by_sample(const SparseShape &s) {
    return s.fc.batch >= kSparseLanesMinBatch && s.fc.n_entries <= 65536;
}

hipError_t launch_fill_sparse_uniform(const SparseShape &s, const float *w, const int32_t *idx,
                                      const int64_t *syn_offsets, const int64_t *in_offsets,
                                      const int32_t *in_pairs, const uint32_t *order, uint32_t n_order,
                                      float *out, bool int_mode, double int_rescaler, Scratch &scr,
                                      hipStream_t st) {
    const uint64_t n = (uint64_t)s.fc.batch * s.fc.n_outputs;
    const int4 *pairs = reinterpret_cast<const int4 *>(in_pairs);
    if (sparse_fill_by_sample(s)) {
        if (s.fc.n_entries <= 256)
            return launch_fill_by_sample<uint8_t>(s, w, idx, in_offsets, pairs, order, n_order, out, int_mode,
                                                  int_rescaler, scr, st);
        return launch_fill_by_sample<uint16_t>(s, w, idx, in_offsets, pairs, order, n_order, out, int_mode,
                                               int_rescaler, scr, st);
    }
    if (scr.mode != Scratch::Run || n == 0) return hipSuccess;
    if (int_mode)
        hipLaunchKernelGGL(k_fill_sparse_uniform<true>, dim3(blocks_for(n)), dim3(kBlock), 0, st,
                           w, idx, syn_offsets, in_offsets, pairs, out, s.fc.batch, s.fc.n_outputs,
                           s.fc.n_detectors, s.fc.n_entries, int_rescaler);
    else
        hipLaunchKernelGGL(k_fill_sparse_uniform<false>, dim3(blocks_for(n)), dim3(kBlock), 0, st,
                           w, idx, syn_offsets, in_offsets, pairs, out, s.fc.batch, s.fc.n_outputs,
                           s.fc.n_detectors, s.fc.n_entries, int_rescaler);
    return hipGetLastError();
}

hipError_t launch_fill_sparse_atomic(const SparseShape &s, const float *w, const int32_t *idx,
                                     const int64_t *syn_offsets, const int32_t *syn_targets,
                                     float *out, bool int_mode, double int_rescaler,
                                     hipStream_t st) {
    const uint64_t n_items = (uint64_t)s.fc.batch * s.fc.n_detectors * s.max_groups;
    if (n_items == 0) return hipSuccess;
    if (int_mode)
        hipLaunchKernelGGL(k_fill_sparse_atomic<true>, dim3(blocks_for(n_items)), dim3(kBlock), 0,
                           st, w, idx, syn_offsets, syn_targets, out, s.fc.n_outputs,
                           s.fc.n_detectors, s.fc.n_entries, s.fc.ogs, s.max_groups, n_items,
                           int_rescaler);
    else
        hipLaunchKernelGGL(k_fill_sparse_atomic<false>, dim3(blocks_for(n_items)), dim3(kBlock), 0,
                           st, w, idx, syn_offsets, syn_targets, out, s.fc.n_outputs,
                           s.fc.n_detectors, s.fc.n_entries, s.fc.ogs, s.max_groups, n_items,
                           int_rescaler);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !int_mode) return e;
    return launch_convert_i2f(out, (uint64_t)s.fc.batch * s.fc.n_outputs, int_rescaler, st);
}

hipError_t launch_propagate_sparse(const SparseShape &s, const float *w, const float *g,
                                   const int32_t *idx, const float *min_deltas,
                                   const int32_t *min_idx, const int32_t *anchors,
                                   const int64_t *syn_offsets, const int32_t *syn_targets,
                                   float *x_grad, bool int_mode, double int_rescaler,
                                   hipStream_t st) {
    const uint64_t n_items = (uint64_t)s.fc.batch * s.fc.n_detectors * s.max_groups;
    if (n_items == 0) return hipSuccess;
    const int2 *ap = reinterpret_cast<const int2 *>(anchors);
    // fp32 sums over uniform rows: slots for the typical group (a median row, at
    // most ogs entries), longer groups take more passes
    const uint32_t span = std::min(s.fc.ogs, s.typ_row);
    const uint64_t n_rows_items = (uint64_t)s.fc.n_detectors * s.max_groups;
    if (!int_mode && s.uniform && s.max_row > 0 && span > 0 && s.fc.batch <= 65535 &&
        n_rows_items * kRowLanes <= 0x7fffffffull) {
        const uint32_t n_x = (uint32_t)n_rows_items;
        const dim3 grid((uint32_t)((n_rows_items * kRowLanes + kBlock - 1) / kBlock), s.fc.batch);
        const uint32_t slots = (span + kRowLanes - 1) / kRowLanes;
        // the LDS sum pays where a sample's adds (two a table and group) come to
        // four or more per input
        const bool red = s.fc.n_inputs <= kRowRedInputs && n_rows_items * 2 >= 4ull * s.fc.n_inputs;
#define SPIKY_PROP_ROWS(P)                                                                                           \
    do {                                                                                                             \
        if (red)                                                                                                     \
            hipLaunchKernelGGL((k_propagate_sparse_rows<P, true>), grid, dim3(kBlock), 0, st, w, g, idx, min_deltas, \
                               min_idx, ap, syn_offsets, syn_targets, x_grad, s.fc.n_inputs, s.fc.n_outputs,         \
                               s.fc.n_detectors, s.fc.n_anchors, s.fc.n_entries, s.fc.ogs, s.max_groups, n_x);       \
        else                                                                                                         \
            hipLaunchKernelGGL((k_propagate_sparse_rows<P, false>), grid, dim3(kBlock), 0, st, w, g, idx,            \
                               min_deltas, min_idx, ap, syn_offsets, syn_targets, x_grad, s.fc.n_inputs,             \
                               s.fc.n_outputs, s.fc.n_detectors, s.fc.n_anchors, s.fc.n_entries, s.fc.ogs,           \
                               s.max_groups, n_x);                                                                   \
    } while (0)
        if (slots <= 1)
            SPIKY_PROP_ROWS(1);
        else if (slots <= 2)
            SPIKY_PROP_ROWS(2);
        else if (slots <= 4)
            SPIKY_PROP_ROWS(4);
        else
            SPIKY_PROP_ROWS(8);
#undef SPIKY_PROP_ROWS
        return hipGetLastError();
    }
    const uint64_t n_threads = n_items * (int_mode ? sp_lanes<true>() : sp_lanes<false>());
    if ((n_threads + kBlock - 1) / kBlock > 0x7fffffffull) return hipErrorInvalidConfiguration;
    if (int_mode)
        hipLaunchKernelGGL(k_propagate_sparse<true>, dim3(blocks_for(n_threads)), dim3(kBlock), 0,
                           st, w, g, idx, min_deltas, min_idx, ap, syn_offsets, syn_targets,
                           x_grad, s.fc.n_inputs, s.fc.n_outputs, s.fc.n_detectors,
                           s.fc.n_anchors, s.fc.n_entries, s.fc.ogs, s.max_groups, n_items,
                           int_rescaler, s.uniform);
    else
        hipLaunchKernelGGL(k_propagate_sparse<false>, dim3(blocks_for(n_threads)), dim3(kBlock), 0,
                           st, w, g, idx, min_deltas, min_idx, ap, syn_offsets, syn_targets,
                           x_grad, s.fc.n_inputs, s.fc.n_outputs, s.fc.n_detectors,
                           s.fc.n_anchors, s.fc.n_entries, s.fc.ogs, s.max_groups, n_items,
                           int_rescaler, s.uniform);
    return hipGetLastError();
}

// scratch: bucket offsets [T][E+1] | sorted samples [T][B]
hipError_t launch_wgrad_sparse(const SparseShape &s, const float *g, const int32_t *idx,
                               const int64_t *syn_offsets, const int32_t *syn_targets,
                               const int32_t *syn_neuron, const int32_t *row_pairs, uint32_t n_row_pairs,
                               float *target, double lr, bool overwrite, bool int_mode, double int_rescaler,
                               Scratch &scratch, uint64_t n_synapses, hipStream_t st) {
    ScratchLayout lay(scratch);
    int32_t *offsets = lay.take<int32_t>((size_t)s.fc.n_detectors * (s.fc.n_entries + 1) * 4);
    int32_t *samples = lay.take<int32_t>((size_t)s.fc.n_detectors * s.fc.batch * 4);
    hipError_t e;
    if (lay.stop(&e, "gather_w_gradients_sparse")) return e;
    if (n_synapses == 0) return hipSuccess;
    e = launch_bucket_samples(s.fc, idx, offsets, samples, st);
    if (e != hipSuccess) return e;
    // the column walk pays where rows average three samples or more (measured
    // on BASELINE config 2: 34 -> 20 us at 4 a row, 14 -> 15 us at 2 a row)
    if (s.uniform && row_pairs && n_row_pairs > 0 && s.fc.batch >= 3u * s.fc.n_entries) {
        const int2 *pairs = reinterpret_cast<const int2 *>(row_pairs);
        // four rows a thread (the fastest of 1..16 at 2 and 4 samples a row)
        const uint32_t rows = std::min(s.fc.n_entries, 4u);
        const uint64_t n_threads = (uint64_t)n_row_pairs * ((s.fc.n_entries + rows - 1) / rows);
        if ((n_threads + kBlock - 1) / kBlock > 0x7fffffffull) return hipErrorInvalidConfiguration;
#define SPIKY_WC(IM, OW)                                                                                      \
    hipLaunchKernelGGL((k_wgrad_sparse_cols<IM, OW>), dim3(blocks_for(n_threads)), dim3(kBlock), 0, st, g,    \
                       offsets, samples, pairs, syn_offsets, syn_targets, target, s.fc.batch, s.fc.n_outputs,   \
                       s.fc.n_entries, n_row_pairs, rows, n_threads, lr, int_rescaler)
        if (int_mode) {
            if (overwrite) SPIKY_WC(true, true); else SPIKY_WC(true, false);
        } else {
            if (overwrite) SPIKY_WC(false, true); else SPIKY_WC(false, false);
        }
#undef SPIKY_WC
        return hipGetLastError();
    }
#define SPIKY_WS(IM, OW)                                                                          \
    hipLaunchKernelGGL((k_wgrad_sparse_rowsum<IM, OW>), dim3(blocks_for(n_synapses)), dim3(kBlock), \
                       0, st, g, offsets, samples, syn_neuron, syn_targets, target, s.fc.batch,   \
                       s.fc.n_outputs, s.fc.n_entries, n_synapses, lr, int_rescaler)
    if (int_mode) {
        if (overwrite) SPIKY_WS(true, true); else SPIKY_WS(true, false);
    } else {
        if (overwrite) SPIKY_WS(false, true); else SPIKY_WS(false, false);
    }
#undef SPIKY_WS
    return hipGetLastError();
}

}  // namespace spiky
