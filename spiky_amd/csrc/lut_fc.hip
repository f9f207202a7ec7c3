// lut_fc.hip -- fully connected LUT layer kernels for gfx950 (CDNA4, wave64).
//
// Data layout in HBM (all row-major, caller-owned):
//   W        fp32 [n_detectors * E][O]      row r = t*E + lookup_index
//   x        fp32 [B][I]
//   anchors  int32 pairs [n_detectors][n_anchors]
//   idx/md/mi [B][n_detectors]
//   out      fp32 [B][O];  x_grad fp32 [B][I];  w_grad like W
//
// Kernels and their schedules:
//   k_check_detectors   one thread per table over the x rows of a few samples
//                       staged in LDS (one thread per (b, t) for very wide x).
//   k_fill_fc           one wavefront per (sample, column slice of 64*VEC);
//                       slices are mapped to XCDs (workgroup id mod 8) so each
//                       XCD's L2 serves one column slice of every table to all
//                       samples; each lane owns VEC columns and walks the tables
//                       in ascending order with fp64 partials per block of `dgs`
//                       tables and an fp32 (or int32) running sum -- the exact
//                       commit order of the reference CPU path, so the output is
//                       bit-identical to it.
//   k_propagate_fc_fast one wavefront per (sample, chunk of tables); chunks are
//                       mapped to XCDs; coalesced float4 reads of the main and
//                       the flipped row, fp64 dot, one pair of fp32 atomics per
//                       (sample, table).
//   k_propagate_fc_exact one thread per (b, t, output block): the reference's
//                       own decomposition, used for int32 summation (its
//                       payloads must be formed per block to stay bit-exact) and
//                       for shapes the fast kernel does not cover.
//   k_bucket_samples +  table-major weight gradient: a stable counting sort of
//   k_wgrad_rowsum      the samples of every table by lookup index, then one
//                       wavefront per table row summing g over its bucket in
//                       ascending sample order (bit-identical to the reference
//                       CPU path) and writing the row once.  No HBM atomics, and
//                       the caller's zero-fill of w_grad can be fused away.
#include "lut_kernels.h"

#include <algorithm>

namespace spiky {
namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return __builtin_amdgcn_readfirstlane(v);
}

__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

// ROUNDED_COMPARISON_GREATER(d, 0.0, cmp_eps), spiky_cuda/misc/misc.h:16
__device__ __forceinline__ bool rounded_greater0(float d, float cmp_eps) {
    if (cmp_eps == 0.0f) return d > 0.0f;
    return (fabsf(d) < cmp_eps) ? false : (d > 0.0f);
}

// du = sign(u) * 0.5 / (1+|u|)^2, sign(u <= 0) = -1, evaluated in the
// reference's order (lut_runtime_kernels_logic.proto:1458-1465).
__device__ __forceinline__ double du_of_margin(float md) {
    double du = (double)md;
    double r = 1.0 / (1.0 + fabs(du));
    return (du > 0) ? r * (0.5 * r) : r * (-0.5 * r);
}

// ---------------------------------------------------------------------------
// check_detectors_logic / check_detectors_eval_logic
// (lut_runtime_kernels_logic.proto:1050-1158).  An anchor id outside
// [0, n_inputs) (including the unused-pair marker -1) is skipped, which is the
// reference's behaviour for the marker and keeps every read in bounds.
// ---------------------------------------------------------------------------
template <bool TRAIN>
__global__ __launch_bounds__(kBlock) void k_check_detectors(
    const float *__restrict__ x, const int2 *__restrict__ anchors, uint32_t n_inputs,
    uint32_t n_detectors, uint32_t n_anchors, uint32_t blocks_per_row, float cmp_eps,
    int32_t *__restrict__ idx, float *__restrict__ md, int32_t *__restrict__ mi) {
    const uint32_t b = blockIdx.x / blocks_per_row;
    const uint32_t t = (blockIdx.x % blocks_per_row) * kBlock + threadIdx.x;
    if (t >= n_detectors) return;
    const float *xb = x + (size_t)b * n_inputs;
    const int2 *ap = anchors + (size_t)t * n_anchors;
    int32_t li = 0;
    float mind = 0.0f;
    int32_t mink = -1;
    for (uint32_t k = 0; k < n_anchors; k++) {
        const int2 a = ap[k];
        if ((uint32_t)a.x >= n_inputs || (uint32_t)a.y >= n_inputs) continue;
        const float d = xb[a.x] - xb[a.y];
        if (rounded_greater0(d, cmp_eps)) li |= (1 << k);
        if (TRAIN) {
            if (mink == -1 || fabsf(d) < fabsf(mind)) {
                mind = d;
                mink = (int32_t)k;
            }
        }
    }
    const size_t o = (size_t)b * n_detectors + t;
    idx[o] = li;
    if (TRAIN) {
        md[o] = mind;
        mi[o] = mink;
    }
}

// The same logic with the x rows of `spb` consecutive samples staged in LDS.
// A thread owns one table: it loads the table's anchor pairs once and
// evaluates them for every staged sample, so the anchor reads are shared by
// spb samples and the 2 * n_anchors input reads per (sample, table) are LDS
// reads instead of dependent global loads.  A workgroup walks `rounds`
// consecutive sample groups with the same anchors in registers, staging each
// group's rows in turn.
constexpr int kCheckMaxAnchors = 16;
constexpr uint32_t kCheckLdsBytes = 64 * 1024;

template <bool TRAIN, int NA>
__global__ __launch_bounds__(1024) void k_check_detectors_lds(
    const float *__restrict__ x, const int2 *__restrict__ anchors, uint32_t batch,
    uint32_t n_inputs, uint32_t n_detectors, uint32_t n_anchors, uint32_t spb, float cmp_eps,
    int32_t *__restrict__ idx, float *__restrict__ md, int32_t *__restrict__ mi, uint32_t gx,
    uint32_t gy, uint32_t rounds) {
    extern __shared__ float xs[];
    // the gx table blocks of one run of sample groups run on one XCD
    // (workgroup i runs on XCD i % 8, consecutively there), so each group's x
    // rows are fetched from HBM once and then served by that XCD's L2
    const uint32_t wl = blockIdx.x;
    const uint32_t run = (wl % 8u) + 8u * (wl / (8u * gx));
    const uint32_t gxb = (wl / 8u) % gx;
    const uint32_t g0 = run * rounds;
    if (g0 >= gy) return;  // uniform over the workgroup
    const uint32_t t = gxb * blockDim.x + threadIdx.x;
    const bool active = t < n_detectors;
    // the table's pairs in registers (fully unrolled, compile-time indices);
    // pairs past n_anchors or with an input id outside [0, n_inputs) are
    // skipped, marked by x = -1
    int2 a[NA];
    const int2 *ap = anchors + (size_t)(active ? t : 0) * n_anchors;
#pragma unroll
    for (int k = 0; k < NA; k++) {
        int2 v = make_int2(-1, -1);
        if ((uint32_t)k < n_anchors) v = ap[k];
        if ((uint32_t)v.x >= n_inputs || (uint32_t)v.y >= n_inputs) v = make_int2(-1, -1);
        a[k] = v;
    }
    const uint32_t g1 = min(g0 + rounds, gy);
    for (uint32_t gyb = g0; gyb < g1; gyb++) {
        const uint32_t b0 = gyb * spb;
        const uint32_t nb = min(spb, batch - b0);
        const uint32_t n_el = nb * n_inputs;
        const float *src = x + (size_t)b0 * n_inputs;
        // every thread is done with the previous group's rows
        if (gyb != g0) __syncthreads();
        if ((n_el & 3u) == 0 && (reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
            const float4 *s4 = reinterpret_cast<const float4 *>(src);
            float4 *d4 = reinterpret_cast<float4 *>(xs);
            for (uint32_t i = threadIdx.x; i < n_el / 4; i += blockDim.x) d4[i] = s4[i];
        } else {
            for (uint32_t i = threadIdx.x; i < n_el; i += blockDim.x) xs[i] = src[i];
        }
        __syncthreads();
        if (!active) continue;
        for (uint32_t sl = 0; sl < nb; sl++) {
            const float *xr = xs + sl * n_inputs;
            int32_t li = 0;
            float mind = 0.0f;
            int32_t mink = -1;
#pragma unroll
            for (int k = 0; k < NA; k++) {
                if (a[k].x >= 0) {
                    const float d = xr[a[k].x] - xr[a[k].y];
                    if (rounded_greater0(d, cmp_eps)) li |= (1 << k);
                    if (TRAIN) {
                        if (mink == -1 || fabsf(d) < fabsf(mind)) {
                            mind = d;
                            mink = (int32_t)k;
                        }
                    }
                }
            }
            const size_t o = (size_t)(b0 + sl) * n_detectors + t;
            idx[o] = li;
            if (TRAIN) {
                md[o] = mind;
                mi[o] = mink;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// fill_outputs_non_seq_fc_logic (proto:1214-1299), re-scheduled.
// ---------------------------------------------------------------------------
template <typename WT, int VEC>
struct RowLoad;

template <>
struct RowLoad<float, 1> {
    __device__ static void load(const float *p, float *v) { v[0] = p[0]; }
};
template <>
struct RowLoad<float, 2> {
    __device__ static void load(const float *p, float *v) {
        const float2 q = *reinterpret_cast<const float2 *>(p);
        v[0] = q.x;
        v[1] = q.y;
    }
};
template <>
struct RowLoad<float, 4> {
    __device__ static void load(const float *p, float *v) {
        const float4 q = *reinterpret_cast<const float4 *>(p);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    }
};
template <>
struct RowLoad<int8_t, 1> {
    __device__ static void load(const int8_t *p, float *v) { v[0] = (float)p[0]; }
};
template <>
struct RowLoad<int8_t, 2> {
    __device__ static void load(const int8_t *p, float *v) {
        const char2 q = *reinterpret_cast<const char2 *>(p);
        v[0] = (float)q.x;
        v[1] = (float)q.y;
    }
};
template <>
struct RowLoad<int8_t, 4> {
    __device__ static void load(const int8_t *p, float *v) {
        const char4 q = *reinterpret_cast<const char4 *>(p);
        v[0] = (float)q.x;
        v[1] = (float)q.y;
        v[2] = (float)q.z;
        v[3] = (float)q.w;
    }
};

// Column slices and XCDs.  A launch covers the outputs in `n_slices` slices of
// 64*VEC columns; workgroup i works on slice i % n_slices.  The hardware hands
// workgroup i to XCD i % 8, so with 8 (or 16) slices every XCD owns whole
// slices and sees every sample's accesses to them: table rows (forward,
// propagate) and gradient rows (weight gradient) are then re-used from that
// XCD's L2 instead of being fetched once per sample from HBM.
constexpr int kWPB = kBlock / kWave;  // wavefronts per workgroup

// Floats per lane such that the slices number at least 8 (one per XCD).
uint32_t pick_vec(uint32_t n_outputs) {
    if (n_outputs % 4 == 0 && n_outputs >= 64u * 4u * 8u) return 4;
    if (n_outputs % 2 == 0 && n_outputs >= 64u * 2u * 8u) return 2;
    return 1;
}

// Forward gather-sum.  Wavefront = SPW samples x one column slice; each lane
// owns VEC columns of every sample and walks the tables in ascending order,
// with an fp64 partial per block of `dgs` tables and an fp32 (or int32) running
// sum -- the reference CPU path's exact commit order, so the output is
// bit-identical to it.  U tables x SPW samples of row loads are issued before
// the ordered adds.  Sample and column indices past the end are clamped to
// valid memory for the loads and masked at the store.
template <typename WT, int VEC, int SPW, int U, bool INT_MODE, bool SCALED>
__global__ __launch_bounds__(kBlock) void k_fill_fc(
    const WT *__restrict__ w, const float *__restrict__ scales, const int32_t *__restrict__ idx,
    float *__restrict__ out, uint32_t batch, uint32_t n_outputs, uint32_t n_detectors,
    uint32_t n_entries, uint32_t dgs, uint32_t n_slices, double int_rescaler) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = uniform(threadIdx.x / kWave);
    const uint32_t slice = blockIdx.x % n_slices;
    const uint32_t b0 = ((blockIdx.x / n_slices) * kWPB + wave) * SPW;
    if (b0 >= batch) return;
    const uint32_t c = (slice * kWave + lane) * VEC;
    const bool active = c < n_outputs;
    const uint32_t cc = active ? c : 0u;
    const uint32_t emask = n_entries - 1;
    const int32_t *ib[SPW];
    bool live[SPW];
#pragma unroll
    for (int s = 0; s < SPW; s++) {
        live[s] = b0 + s < batch;
        ib[s] = idx + (size_t)(live[s] ? b0 + s : b0) * n_detectors;
    }

    float run[SPW][VEC];
    int32_t irun[SPW][VEC];
#pragma unroll
    for (int s = 0; s < SPW; s++) {
#pragma unroll
        for (int v = 0; v < VEC; v++) {
            run[s][v] = 0.0f;
            irun[s][v] = 0;
            if (active && live[s]) {
                const float o = out[(size_t)(b0 + s) * n_outputs + c + v];
                if (INT_MODE)
                    irun[s][v] = __float_as_int(o);
                else
                    run[s][v] = o;
            }
        }
    }

    for (uint32_t t0 = 0; t0 < n_detectors; t0 += dgs) {
        const uint32_t t1 = min(t0 + dgs, n_detectors);
        double acc[SPW][VEC];
#pragma unroll
        for (int s = 0; s < SPW; s++)
#pragma unroll
            for (int v = 0; v < VEC; v++) acc[s][v] = 0.0;
        uint32_t t = t0;
        for (; t + U <= t1; t += U) {
            float vals[U][SPW][VEC];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const WT *wt = w + (size_t)(t + u) * n_entries * n_outputs + cc;
#pragma unroll
                for (int s = 0; s < SPW; s++) {
                    const uint32_t r = (uint32_t)ib[s][t + u] & emask;
                    RowLoad<WT, VEC>::load(wt + (size_t)r * n_outputs, vals[u][s]);
                }
                if (SCALED) {
                    const float sc = scales[t + u];
#pragma unroll
                    for (int s = 0; s < SPW; s++)
#pragma unroll
                        for (int v = 0; v < VEC; v++) vals[u][s][v] = sc * vals[u][s][v];
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int s = 0; s < SPW; s++)
#pragma unroll
                    for (int v = 0; v < VEC; v++) acc[s][v] += (double)vals[u][s][v];
        }
        for (; t < t1; t++) {
            const WT *wt = w + (size_t)t * n_entries * n_outputs + cc;
            float vals[SPW][VEC];
#pragma unroll
            for (int s = 0; s < SPW; s++) {
                const uint32_t r = (uint32_t)ib[s][t] & emask;
                RowLoad<WT, VEC>::load(wt + (size_t)r * n_outputs, vals[s]);
            }
            const float sc = SCALED ? scales[t] : 1.0f;
#pragma unroll
            for (int s = 0; s < SPW; s++)
#pragma unroll
                for (int v = 0; v < VEC; v++)
                    acc[s][v] += (double)(SCALED ? sc * vals[s][v] : vals[s][v]);
        }
#pragma unroll
        for (int s = 0; s < SPW; s++)
#pragma unroll
            for (int v = 0; v < VEC; v++) {
                if (INT_MODE)
                    irun[s][v] = wrap_add(irun[s][v], (int32_t)(acc[s][v] * kDenom32 * int_rescaler));
                else
                    run[s][v] += (float)acc[s][v];
            }
    }
    if (!active) return;
#pragma unroll
    for (int s = 0; s < SPW; s++) {
        if (!live[s]) continue;
        float *ob = out + (size_t)(b0 + s) * n_outputs + c;
#pragma unroll
        for (int v = 0; v < VEC; v++) {
            if (INT_MODE) {
                // convert_integers_to_floats_logic, proto:200-213
                const double y = (double)irun[s][v] * kDenom32Reciproc;
                ob[v] = (float)(y / int_rescaler);
            } else {
                ob[v] = run[s][v];
            }
        }
    }
}

template <typename WT, int VEC, bool INT_MODE, bool SCALED>
hipError_t launch_fill_variant(const FcShape &s, const WT *w, const float *scales,
                               const int32_t *idx, float *out, double int_rescaler,
                               hipStream_t st) {
    const uint32_t n_slices = (s.n_outputs + kWave * VEC - 1) / (kWave * VEC);
    // several samples per wavefront once the batch is large enough to fill the chip
    const uint32_t spw = s.batch >= 512 ? 4 : 1;
    const uint32_t b_groups = (s.batch + kWPB * spw - 1) / (kWPB * spw);
    const uint64_t grid = (uint64_t)n_slices * b_groups;
    if (grid == 0) return hipSuccess;
    if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
    if (spw == 4)
        hipLaunchKernelGGL((k_fill_fc<WT, VEC, 4, 8, INT_MODE, SCALED>), dim3((uint32_t)grid),
                           dim3(kBlock), 0, st, w, scales, idx, out, s.batch, s.n_outputs,
                           s.n_detectors, s.n_entries, s.dgs, n_slices, int_rescaler);
    else
        hipLaunchKernelGGL((k_fill_fc<WT, VEC, 1, 16, INT_MODE, SCALED>), dim3((uint32_t)grid),
                           dim3(kBlock), 0, st, w, scales, idx, out, s.batch, s.n_outputs,
                           s.n_detectors, s.n_entries, s.dgs, n_slices, int_rescaler);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// propagate_through_detectors_non_seq_fc_logic (proto:1421-1499), exact form:
// one thread per (b, t, output block), fp64 dots in ascending output order.
// ---------------------------------------------------------------------------
template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_propagate_fc_exact(
    const float *__restrict__ w, const float *__restrict__ g, const int32_t *__restrict__ idx,
    const float *__restrict__ md, const int32_t *__restrict__ mi, const int2 *__restrict__ anchors,
    float *__restrict__ x_grad, uint32_t n_inputs, uint32_t n_outputs, uint32_t n_detectors,
    uint32_t n_anchors, uint32_t n_entries, uint32_t ogs, uint32_t n_ob, uint64_t n_items,
    double int_rescaler) {
    const uint64_t item = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (item >= n_items) return;
    const uint64_t per_b = (uint64_t)n_detectors * n_ob;
    const uint32_t b = (uint32_t)(item / per_b);
    const uint32_t rem = (uint32_t)(item % per_b);
    const uint32_t t = rem / n_ob;
    const uint32_t ob = rem % n_ob;
    const size_t bt = (size_t)b * n_detectors + t;
    const int32_t m = mi[bt];
    if (m < 0 || (uint32_t)m >= n_anchors) return;
    const uint32_t r = (uint32_t)idx[bt] & (n_entries - 1);
    const uint32_t ra = r ^ (1u << m);
    double du = du_of_margin(md[bt]);
    const uint32_t o0 = ob * ogs;
    const uint32_t o1 = min(o0 + ogs, n_outputs);
    const float *wm = w + ((size_t)t * n_entries + r) * n_outputs;
    const float *wa = w + ((size_t)t * n_entries + ra) * n_outputs;
    const float *gb = g + (size_t)b * n_outputs;
    double ms = 0.0, as = 0.0;
    for (uint32_t o = o0; o < o1; o++) {
        const double gg = (double)gb[o];
        ms += (double)wm[o] * gg;
        as += (double)wa[o] * gg;
    }
    du *= ms - as;
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

// ---------------------------------------------------------------------------
// propagate, fp32-summation form over column slices.  Wavefront = SPW samples
// x one column slice (slice -> XCD as in the forward).  For every (sample,
// table) the lane-partial fp64 dot  sum_c (W_main[c] - W_alt[c]) * g[c]  over
// the slice is reduced across the wavefront, scaled by du(min margin), and
// committed as one pair of fp32 atomics per (sample, table, slice).  The
// reference commits one pair per 32-output block (forward_group_size); the
// slice commit differs from it only in fp32 rounding of the committed terms.
// ---------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <int VEC, int SPW, int U>
__global__ __launch_bounds__(kBlock) void k_propagate_fc_slices(
    const float *__restrict__ w, const float *__restrict__ g, const int32_t *__restrict__ idx,
    const float *__restrict__ md, const int32_t *__restrict__ mi, const int2 *__restrict__ anchors,
    float *__restrict__ x_grad, uint32_t batch, uint32_t n_inputs, uint32_t n_outputs,
    uint32_t n_detectors, uint32_t n_anchors, uint32_t n_entries, uint32_t n_slices) {
    static_assert(U * SPW <= kWave, "one committing lane per (sample, table)");
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = uniform(threadIdx.x / kWave);
    const uint32_t slice = blockIdx.x % n_slices;
    const uint32_t b0 = ((blockIdx.x / n_slices) * kWPB + wave) * SPW;
    if (b0 >= batch) return;
    const uint32_t c = (slice * kWave + lane) * VEC;
    const bool active = c < n_outputs;
    const uint32_t cc = active ? c : 0u;
    const uint32_t emask = n_entries - 1;

    uint32_t bs[SPW];
    double gd[SPW][VEC];
#pragma unroll
    for (int s = 0; s < SPW; s++) {
        bs[s] = (b0 + s < batch) ? b0 + s : b0;
        float gv[VEC];
        RowLoad<float, VEC>::load(g + (size_t)bs[s] * n_outputs + cc, gv);
#pragma unroll
        for (int v = 0; v < VEC; v++) gd[s][v] = active ? (double)gv[v] : 0.0;
    }
    // the committing lane j = u*SPW + s handles (sample b0+s, table t+u)
    const uint32_t my_s = lane % SPW;
    const uint32_t my_u = lane / SPW;
    const bool my_live = lane < (uint32_t)(U * SPW) && b0 + my_s < batch;
    const uint32_t my_b = b0 + (my_live ? my_s : 0u);

    for (uint32_t t = 0; t < n_detectors; t += U) {
        float mv[U][SPW][VEC], av[U][SPW][VEC];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t tt = min(t + u, n_detectors - 1);
            const float *wt = w + (size_t)tt * n_entries * n_outputs + cc;
#pragma unroll
            for (int s = 0; s < SPW; s++) {
                const size_t bt = (size_t)bs[s] * n_detectors + tt;
                const int32_t m = mi[bt];
                const uint32_t r = (uint32_t)idx[bt] & emask;
                const uint32_t ra = (m >= 0 && (uint32_t)m < n_anchors) ? (r ^ (1u << m)) : r;
                RowLoad<float, VEC>::load(wt + (size_t)r * n_outputs, mv[u][s]);
                RowLoad<float, VEC>::load(wt + (size_t)ra * n_outputs, av[u][s]);
            }
        }
        double mine = 0.0;
#pragma unroll
        for (int u = 0; u < U; u++) {
#pragma unroll
            for (int s = 0; s < SPW; s++) {
                double p = 0.0;
#pragma unroll
                for (int v = 0; v < VEC; v++)
                    p += ((double)mv[u][s][v] - (double)av[u][s][v]) * gd[s][v];
                p = wave_sum(p);
                if (lane == (uint32_t)(u * SPW + s)) mine = p;
            }
        }
        const uint32_t my_t = t + my_u;
        if (my_live && my_t < n_detectors) {
            const size_t bt = (size_t)my_b * n_detectors + my_t;
            const int32_t m = mi[bt];
            if (m >= 0 && (uint32_t)m < n_anchors) {
                const double du = du_of_margin(md[bt]) * mine;
                if (fabs(du) > kEps) {
                    const int2 a = anchors[(size_t)my_t * n_anchors + m];
                    if ((uint32_t)a.x < n_inputs && (uint32_t)a.y < n_inputs) {
                        float *xg = x_grad + (size_t)my_b * n_inputs;
                        unsafeAtomicAdd(xg + a.x, (float)du);
                        unsafeAtomicAdd(xg + a.y, (float)(-du));
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// gather_w_gradients_non_seq_fc_logic (proto:1547-1585), generic atomic form:
// one thread per (b, t, o).
// ---------------------------------------------------------------------------
template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_wgrad_fc_atomic(
    const float *__restrict__ g, const int32_t *__restrict__ idx, float *__restrict__ target,
    uint32_t n_outputs, uint32_t n_detectors, uint32_t n_entries, uint64_t n_items, double lr,
    double int_rescaler) {
    const uint64_t item = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (item >= n_items) return;
    const uint32_t o = (uint32_t)(item % n_outputs);
    const uint64_t bt = item / n_outputs;
    const uint32_t t = (uint32_t)(bt % n_detectors);
    const uint32_t b = (uint32_t)(bt / n_detectors);
    const double gg = (double)g[(size_t)b * n_outputs + o];
    if (!(fabs(gg) > kEps)) return;
    const uint32_t r = (uint32_t)idx[bt] & (n_entries - 1);
    float *p = target + ((size_t)t * n_entries + r) * n_outputs + o;
    if (INT_MODE)
        atomicAdd(reinterpret_cast<int32_t *>(p), (int32_t)(gg * lr * kDenom32 * int_rescaler));
    else
        unsafeAtomicAdd(p, (float)(gg * lr));
}

// ---------------------------------------------------------------------------
// Stable counting sort of samples by lookup index, one wavefront per table.
// offsets[t][e] .. offsets[t][e+1] delimit bucket e in samples[t][*], and the
// samples of a bucket are in ascending order.
// ---------------------------------------------------------------------------
// The lookup indices come from idx [B][T] (a strided column per table) or, when
// key_t is given, from the transposed keys [T][key_pitch] that the table-major
// propagate writes (main << key_shift | (alternative << key_shift) << 16): one
// contiguous row per table.
__global__ __launch_bounds__(kWave) void k_bucket_samples(
    const int32_t *__restrict__ idx, const uint32_t *__restrict__ key_t, uint32_t key_pitch,
    uint32_t key_shift, uint32_t batch, uint32_t n_detectors, uint32_t n_entries, uint32_t n_bits,
    int32_t *__restrict__ offsets, int32_t *__restrict__ samples) {
    extern __shared__ int32_t cnt[];
    const uint32_t t = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const uint32_t emask = n_entries - 1;
    const uint32_t *kt = key_t ? key_t + (size_t)t * key_pitch : nullptr;
    auto key_of = [&](uint32_t b) -> uint32_t {
        return kt ? (((kt[b] & 0xFFFFu) >> key_shift) & emask) : ((uint32_t)idx[(size_t)b * n_detectors + t] & emask);
    };
    // up to kBsCache keys a lane stay in registers for both passes, all loaded
    // up front (a batch of at most 64 * kBsCache samples)
    constexpr int kBsCache = 16;
    const bool cached = batch <= (uint32_t)(kWave * kBsCache);
    uint32_t kc[kBsCache];
    if (cached) {
#pragma unroll
        for (int u = 0; u < kBsCache; u++) {
            const uint32_t b = u * kWave + lane;
            kc[u] = b < batch ? key_of(b) : 0u;
        }
    }
    for (uint32_t e = lane; e < n_entries; e += kWave) cnt[e] = 0;
    __syncthreads();
    if (cached) {
#pragma unroll
        for (int u = 0; u < kBsCache; u++)
            if (u * kWave + lane < batch) atomicAdd(&cnt[kc[u]], 1);
    } else {
        for (uint32_t base = 0; base < batch; base += kWave) {
            const uint32_t b = base + lane;
            if (b < batch) atomicAdd(&cnt[key_of(b)], 1);
        }
    }
    __syncthreads();
    // exclusive scan of cnt[0..E) by one wavefront: each lane sums a contiguous run
    const uint32_t per_lane = (n_entries + kWave - 1) / kWave;
    const uint32_t e0 = min(lane * per_lane, n_entries);
    const uint32_t e1 = min(e0 + per_lane, n_entries);
    int32_t local = 0;
    for (uint32_t e = e0; e < e1; e++) local += cnt[e];
    int32_t incl = local;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int32_t y = __shfl_up(incl, off, kWave);
        if ((int)lane >= off) incl += y;
    }
    int32_t run = incl - local;
    __syncthreads();
    int32_t *off_t = offsets + (size_t)t * (n_entries + 1);
    for (uint32_t e = e0; e < e1; e++) {
        const int32_t c = cnt[e];
        cnt[e] = run;
        off_t[e] = run;
        run += c;
    }
    if (lane == kWave - 1) off_t[n_entries] = incl;
    __syncthreads();
    int32_t *smp_t = samples + (size_t)t * batch;
    // samples base .. base + 63 in order: ballot-ranked among equal keys
    auto scatter = [&](uint32_t base, uint32_t key) {
        const uint32_t b = base + lane;
        const bool valid = b < batch;
        uint64_t peers = __ballot(valid);
        for (uint32_t bit = 0; bit < n_bits; bit++) {
            const bool kb = (key >> bit) & 1u;
            const uint64_t bm = __ballot(kb);
            peers &= kb ? bm : ~bm;
        }
        const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
        const int32_t rank = __popcll(peers & lt);
        int32_t pos = 0;
        if (valid) pos = cnt[key] + rank;
        __syncthreads();
        if (valid) {
            smp_t[pos] = (int32_t)b;
            const uint32_t leader = 63u - (uint32_t)__clzll(peers);
            if (lane == leader) cnt[key] = pos + 1;
        }
        __syncthreads();
    };
    if (cached) {
#pragma unroll
        for (int u = 0; u < kBsCache; u++) {
            if ((uint32_t)u * kWave >= batch) break;  // uniform
            scatter((uint32_t)u * kWave, kc[u]);
        }
    } else {
        for (uint32_t base = 0; base < batch; base += kWave)
            scatter(base, base + lane < batch ? key_of(base + lane) : 0u);
    }
}

// The same sort with a 1024-thread workgroup per table, for few tables over
// many samples (the sequence layers: 16-64 tables of 8192 (b, s) rows).  Wave w
// takes a contiguous run of the samples; per-wave bucket counts (LDS) are
// scanned in (bucket, wave) order, so every wave knows where its run of each
// bucket starts, and the waves scatter their runs in sample order: the result
// equals the one-wavefront sort's.
constexpr int kBsThreads = 1024;
constexpr int kBsWaves = kBsThreads / kWave;
constexpr uint32_t kBsMaxEntries = 1024;

__global__ __launch_bounds__(kBsThreads) void k_bucket_samples_wg(
    const int32_t *__restrict__ idx, const uint32_t *__restrict__ key_t, uint32_t key_pitch,
    uint32_t key_shift, uint32_t batch, uint32_t n_detectors, uint32_t n_entries, uint32_t n_bits,
    int32_t *__restrict__ offsets, int32_t *__restrict__ samples) {
    extern __shared__ int32_t hist[];  // [kBsWaves][n_entries]
    __shared__ int32_t wsum[kBsWaves];
    const uint32_t t = blockIdx.x;
    const uint32_t tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const uint32_t emask = n_entries - 1;
    const uint32_t *kt = key_t ? key_t + (size_t)t * key_pitch : nullptr;
    auto key_of = [&](uint32_t b) -> uint32_t {
        return kt ? (((kt[b] & 0xFFFFu) >> key_shift) & emask) : ((uint32_t)idx[(size_t)b * n_detectors + t] & emask);
    };
    // this wave's run of samples: whole 64-sample groups
    const uint32_t groups = (batch + kWave - 1) / kWave;
    const uint32_t per = (groups + kBsWaves - 1) / kBsWaves;
    const uint32_t r0 = min(wave * per * kWave, batch), r1 = min(r0 + per * kWave, batch);
    int32_t *h = hist + wave * n_entries;
    for (uint32_t e = lane; e < n_entries; e += kWave) h[e] = 0;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
    // lanes with the same key in a group of 64 samples, and this lane's rank among them
    auto peers_of = [&](uint32_t key, bool valid) -> uint64_t {
        uint64_t peers = __ballot(valid);
        for (uint32_t bit = 0; bit < n_bits; bit++) {
            const bool kb = (key >> bit) & 1u;
            const uint64_t bm = __ballot(kb);
            peers &= kb ? bm : ~bm;
        }
        return peers;
    };
    for (uint32_t base = r0; base < r1; base += kWave) {
        const uint32_t b = base + lane;
        const bool valid = b < r1;
        const uint32_t key = valid ? key_of(b) : 0u;
        const uint64_t peers = peers_of(key, valid);
        if (valid && lane == 63u - (uint32_t)__clzll(peers)) h[key] += __popcll(peers);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __syncthreads();
    // bucket e's runs: exclusive prefix over the waves, then over the buckets
    int32_t tot = 0;
    if (tid < n_entries) {
        for (uint32_t w = 0; w < (uint32_t)kBsWaves; w++) {
            const int32_t c = hist[w * n_entries + tid];
            hist[w * n_entries + tid] = tot;
            tot += c;
        }
    }
    int32_t incl = tot;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int32_t y = __shfl_up(incl, off, kWave);
        if ((int)lane >= off) incl += y;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int32_t before = 0;
    for (uint32_t w = 0; w < wave; w++) before += wsum[w];
    int32_t *off_t = offsets + (size_t)t * (n_entries + 1);
    if (tid < n_entries) {
        const int32_t start = before + incl - tot;
        off_t[tid] = start;
        for (uint32_t w = 0; w < (uint32_t)kBsWaves; w++) hist[w * n_entries + tid] += start;
    }
    if (tid == 0) off_t[n_entries] = (int32_t)batch;
    __syncthreads();
    int32_t *smp_t = samples + (size_t)t * batch;
    for (uint32_t base = r0; base < r1; base += kWave) {
        const uint32_t b = base + lane;
        const bool valid = b < r1;
        const uint32_t key = valid ? key_of(b) : 0u;
        const uint64_t peers = peers_of(key, valid);
        if (valid) {
            smp_t[h[key] + __popcll(peers & lt)] = (int32_t)b;
            if (lane == 63u - (uint32_t)__clzll(peers)) h[key] += __popcll(peers);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Commit values of the weight gradient, one per (sample, output): what the
// reference adds to a table row for that sample (gather_weight_gradients_fc,
// proto:731-790): (float)((double)g * lr) if |(double)g| > EPS, or the int32
// payload (int32)(g * lr * DENOM32 * int_rescaler) for int32 summation.  A
// skipped term becomes -0.0f (float) or 0 (int), which leaves any sum
// unchanged bit for bit (x + -0.0f == x for every x, including +-0.0).
template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_wgrad_commit_values(
    const float *__restrict__ g, uint32_t *__restrict__ cv, uint64_t n, double lr,
    double int_rescaler) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const double gg = (double)g[i];
    uint32_t v;
    if (INT_MODE)
        v = fabs(gg) > kEps ? (uint32_t)(int32_t)(gg * lr * kDenom32 * int_rescaler) : 0u;
    else
        v = fabs(gg) > kEps ? __float_as_uint((float)(gg * lr)) : 0x80000000u;
    cv[i] = v;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int VEC>
struct CvLoad;
template <>
struct CvLoad<1> {
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint32_t *v) {
        v[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
    }
};
template <>
struct CvLoad<2> {
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint32_t *v) {
        const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
        v[0] = q.x;
        v[1] = q.y;
    }
};
template <>
struct CvLoad<4> {
    __device__ static void load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, uint32_t *v) {
        const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    }
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Non-temporal store of VEC floats (one instruction).
template <int VEC>
struct NtStore;
template <>
struct NtStore<1> {
    __device__ static void store(float *p, const float *v) { __builtin_nontemporal_store(v[0], p); }
};
template <>
struct NtStore<2> {
    __device__ static void store(float *p, const float *v) {
        __builtin_nontemporal_store(f32x2{v[0], v[1]}, reinterpret_cast<f32x2 *>(p));
    }
};
template <>
struct NtStore<4> {
    __device__ static void store(float *p, const float *v) {
        __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4 *>(p));
    }
};

// Table-major weight gradient over column slices.  Wavefront = `rpw` (<= 63)
// consecutive rows of one table x one column slice (slice -> XCD, so each XCD
// only ever reads its own column slice of the commit values, which stays in its
// L2).  The rows' buckets are contiguous in the table's sorted sample list, so
// the wavefront walks that list in batches of KB samples (the next batch
// loading while the current one is added, ping-pong) and closes a row whenever
// the walk crosses its bucket end.  Within a row the commit values are added in
// ascending sample order into an fp32 (or int32) sum starting from the target
// value (or zero when overwriting): the reference CPU path's order, so the
// result is bit-identical to it, and each target element is written exactly
// once with no atomics.  Commit-value rows are read with buffer loads whose row
// offset is a scalar register, so a sample costs VEC adds and one lane read.
template <int VEC, int KB, bool INT_MODE, bool OVERWRITE>
__global__ __launch_bounds__(kBlock) void k_wgrad_slices(
    const uint32_t *__restrict__ cv, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ samples, float *__restrict__ target, uint32_t batch,
    uint32_t n_outputs, uint32_t n_entries, uint32_t n_detectors, uint32_t n_slices, uint32_t rpw,
    double int_rescaler) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = uniform(threadIdx.x / kWave);
    const uint32_t slice = blockIdx.x % n_slices;
    const uint64_t unit = (uint64_t)(blockIdx.x / n_slices) * kWPB + wave;
    const uint32_t groups = n_entries / rpw;
    const uint64_t t64 = unit / groups;
    if (t64 >= n_detectors) return;
    const uint32_t t = (uint32_t)t64;
    const uint32_t e0 = (uint32_t)(unit % groups) * rpw;
    const uint32_t c = (slice * kWave + lane) * VEC;
    const bool active = c < n_outputs;
    const uint32_t cc = active ? c : 0u;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)cv, (short)0, (int)(batch * n_outputs * 4u), 0x00020000);
    const uint32_t voff = cc * 4u;
    const uint32_t row_bytes = n_outputs * 4u;

    // lane i <= rpw holds the start of bucket e0 + i
    const int32_t *off_t = offsets + (size_t)t * (n_entries + 1) + e0;
    const int32_t offv = lane <= rpw ? off_t[lane] : 0;
    const int32_t *smp = samples + (size_t)t * batch;
    float *tb = target + ((size_t)t * n_entries + e0) * n_outputs + cc;
    const int32_t kbeg = __builtin_amdgcn_readfirstlane(offv);
    const int32_t kend = __builtin_amdgcn_readlane(offv, rpw);

    uint32_t acc[VEC];
    auto init = [&](uint32_t e) {
#pragma unroll
        for (int q = 0; q < VEC; q++) acc[q] = 0u;  // +0.0f / int 0
        if (!OVERWRITE) {
            float v[VEC];
            RowLoad<float, VEC>::load(tb + (size_t)e * n_outputs, v);
#pragma unroll
            for (int q = 0; q < VEC; q++) acc[q] = __float_as_uint(v[q]);
        }
    };
    // the rows are written once and not re-read here: non-temporal stores keep
    // them from evicting the commit values this XCD re-reads from its L2
    auto store = [&](uint32_t e) {
        if (!active) return;
        float *p = tb + (size_t)e * n_outputs;
        float v[VEC];
#pragma unroll
        for (int q = 0; q < VEC; q++)
            v[q] = INT_MODE ? (float)(((double)(int32_t)acc[q] * kDenom32Reciproc) / int_rescaler)
                            : __uint_as_float(acc[q]);
        NtStore<VEC>::store(p, v);
    };

    uint32_t e = 0;
    int32_t row_end = __builtin_amdgcn_readlane(offv, 1);
    init(0);
    for (int32_t k = kbeg; k < kend; k += kWave) {
        const int32_t n = min((int32_t)kWave, kend - k);
        const int32_t idv = smp[k + min((int32_t)lane, n - 1)];
        uint32_t va[KB][VEC], vb[KB][VEC];
        auto load = [&](uint32_t (&v)[KB][VEC], int32_t j0) {
#pragma unroll
            for (int j = 0; j < KB; j++) {
                const uint32_t b = (uint32_t)__builtin_amdgcn_readlane(idv, min(j0 + j, n - 1));
                CvLoad<VEC>::load(rsrc, voff, b * row_bytes, v[j]);
            }
        };
        auto add = [&](const uint32_t (&v)[KB][VEC], int32_t j0) {
#pragma unroll
            for (int j = 0; j < KB; j++) {
                if (j0 + j >= n) break;
                const int32_t kk = k + j0 + j;
                while (kk >= row_end) {
                    store(e);
                    e++;
                    row_end = __builtin_amdgcn_readlane(offv, e + 1);
                    init(e);
                }
#pragma unroll
                for (int q = 0; q < VEC; q++) {
                    if (INT_MODE)
                        acc[q] = acc[q] + v[j][q];
                    else
                        acc[q] = __float_as_uint(__uint_as_float(acc[q]) + __uint_as_float(v[j][q]));
                }
            }
        };
        int32_t j0 = 0;
        load(va, 0);
        for (;;) {
            const bool more_b = j0 + KB < n;
            if (more_b) load(vb, j0 + KB);
            add(va, j0);
            j0 += KB;
            if (!more_b) break;
            const bool more_a = j0 + KB < n;
            if (more_a) load(va, j0 + KB);
            add(vb, j0);
            j0 += KB;
            if (!more_a) break;
        }
    }
    for (;;) {
        store(e);
        e++;
        if (e >= rpw) break;
        init(e);
    }
}

__global__ __launch_bounds__(kBlock) void k_zero(float *__restrict__ buf, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n) buf[i] = 0.0f;
}

__global__ __launch_bounds__(kBlock) void k_convert_i2f(float *__restrict__ buf, uint64_t n,
                                                        double int_rescaler) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const double y = (double)__float_as_int(buf[i]) * kDenom32Reciproc;
    buf[i] = (float)(y / int_rescaler);
}

uint32_t blocks_for(uint64_t n) { return (uint32_t)((n + kBlock - 1) / kBlock); }

// The bucketed weight gradient needs the per-table bucket counters in LDS and
// byte offsets of the commit values within 32 bits (buffer loads).
bool rowsum_applies(const FcShape &s) {
    return s.n_entries <= 4096 && (uint64_t)s.batch * s.n_outputs * 4 < 0x7fffffffull;
}

}  // namespace

// ---------------------------------------------------------------------------
hipError_t launch_check_detectors(const FcShape &s, const float *x, const int32_t *anchors,
                                  float cmp_eps, int32_t *idx, float *min_deltas,
                                  int32_t *min_idx, hipStream_t st) {
    if ((uint64_t)s.batch * s.n_detectors == 0) return hipSuccess;
    const int2 *ap = reinterpret_cast<const int2 *>(anchors);
    const uint32_t spb_lds = kCheckLdsBytes / 4 / std::max<uint32_t>(s.n_inputs, 1);
    if (s.n_anchors <= (uint32_t)kCheckMaxAnchors && spb_lds >= 1 &&
        (uint64_t)(s.batch + 7) * ((s.n_detectors + 63) / 64) <= 0x7fffffffull) {
        // one thread per table, x rows of spb samples in LDS; spb is lowered so
        // that the grid still holds ~512 workgroups where the batch allows it
        const uint32_t threads = std::min<uint32_t>(1024, (s.n_detectors + 63) / 64 * 64);
        const uint32_t gx = (s.n_detectors + threads - 1) / threads;
        const uint64_t want = std::max<uint64_t>(1, (uint64_t)s.batch * gx / 512);
        const uint32_t spb = (uint32_t)std::min<uint64_t>({(uint64_t)spb_lds, want, 16});
        const uint32_t gy = (s.batch + spb - 1) / spb;
        // sample groups a workgroup walks: enough to leave ~512 workgroups
        const uint32_t rounds = (uint32_t)std::max<uint64_t>(1, (uint64_t)gy * gx / 512);
        const uint32_t runs = (gy + rounds - 1) / rounds;
        const uint64_t grid = 8ull * gx * ((runs + 7) / 8);
        if (grid > 0x7fffffffull) return hipErrorInvalidConfiguration;
        const size_t lds = (size_t)spb * s.n_inputs * sizeof(float);
#define SPIKY_CHK(TR, NA)                                                                       \
    hipLaunchKernelGGL((k_check_detectors_lds<TR, NA>), dim3((uint32_t)grid), dim3(threads), lds, st, x, \
                       ap, s.batch, s.n_inputs, s.n_detectors, s.n_anchors, spb, cmp_eps, idx,   \
                       min_deltas, min_idx, gx, gy, rounds)
        if (min_deltas) {
            if (s.n_anchors <= 8) SPIKY_CHK(true, 8); else SPIKY_CHK(true, 16);
        } else {
            if (s.n_anchors <= 8) SPIKY_CHK(false, 8); else SPIKY_CHK(false, 16);
        }
#undef SPIKY_CHK
        return hipGetLastError();
    }
    const uint32_t bpr = (s.n_detectors + kBlock - 1) / kBlock;
    const uint64_t grid = (uint64_t)bpr * s.batch;
    if (min_deltas)
        hipLaunchKernelGGL(k_check_detectors<true>, dim3((uint32_t)grid), dim3(kBlock), 0, st, x,
                           ap, s.n_inputs, s.n_detectors, s.n_anchors, bpr, cmp_eps, idx,
                           min_deltas, min_idx);
    else
        hipLaunchKernelGGL(k_check_detectors<false>, dim3((uint32_t)grid), dim3(kBlock), 0, st, x,
                           ap, s.n_inputs, s.n_detectors, s.n_anchors, bpr, cmp_eps, idx,
                           (float *)nullptr, (int32_t *)nullptr);
    return hipGetLastError();
}

hipError_t launch_fill_fc_f32(const FcShape &s, const float *w, const int32_t *idx, float *out,
                              bool int_mode, double int_rescaler, hipStream_t st) {
#define SPIKY_FILL_F32(V)                                                                        \
    return int_mode ? launch_fill_variant<float, V, true, false>(s, w, nullptr, idx, out,        \
                                                                 int_rescaler, st)               \
                    : launch_fill_variant<float, V, false, false>(s, w, nullptr, idx, out,       \
                                                                  int_rescaler, st)
    switch (pick_vec(s.n_outputs)) {
        case 4: SPIKY_FILL_F32(4);
        case 2: SPIKY_FILL_F32(2);
        default: SPIKY_FILL_F32(1);
    }
#undef SPIKY_FILL_F32
}

hipError_t launch_fill_fc_i8(const FcShape &s, const int8_t *q8, const float *scales,
                             const int32_t *idx, float *out, bool int_mode, double int_rescaler,
                             hipStream_t st) {
#define SPIKY_FILL_I8(V)                                                                         \
    return int_mode ? launch_fill_variant<int8_t, V, true, true>(s, q8, scales, idx, out,        \
                                                                 int_rescaler, st)               \
                    : launch_fill_variant<int8_t, V, false, true>(s, q8, scales, idx, out,       \
                                                                  int_rescaler, st)
    switch (pick_vec(s.n_outputs)) {
        case 4: SPIKY_FILL_I8(4);
        case 2: SPIKY_FILL_I8(2);
        default: SPIKY_FILL_I8(1);
    }
#undef SPIKY_FILL_I8
}

hipError_t launch_propagate_fc(const FcShape &s, const float *w, const float *g,
                               const int32_t *idx, const float *min_deltas,
                               const int32_t *min_idx, const int32_t *anchors, float *x_grad,
                               bool int_mode, double int_rescaler, hipStream_t st) {
    const int2 *ap = reinterpret_cast<const int2 *>(anchors);
    if (!int_mode && s.n_outputs >= 256) {
        const uint32_t vec = pick_vec(s.n_outputs);
        const uint32_t n_slices = (s.n_outputs + kWave * vec - 1) / (kWave * vec);
        const uint32_t spw = s.batch >= 512 ? 4 : 1;
        const uint32_t b_groups = (s.batch + kWPB * spw - 1) / (kWPB * spw);
        const uint64_t grid = (uint64_t)n_slices * b_groups;
        if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
#define SPIKY_PROP(V, SPW, U)                                                                     \
    hipLaunchKernelGGL((k_propagate_fc_slices<V, SPW, U>), dim3((uint32_t)grid), dim3(kBlock), 0, \
                       st, w, g, idx, min_deltas, min_idx, ap, x_grad, s.batch, s.n_inputs,       \
                       s.n_outputs, s.n_detectors, s.n_anchors, s.n_entries, n_slices)
        if (spw == 4) {
            switch (vec) {
                case 4: SPIKY_PROP(4, 4, 4); break;
                case 2: SPIKY_PROP(2, 4, 4); break;
                default: SPIKY_PROP(1, 4, 4); break;
            }
        } else {
            switch (vec) {
                case 4: SPIKY_PROP(4, 1, 8); break;
                case 2: SPIKY_PROP(2, 1, 8); break;
                default: SPIKY_PROP(1, 1, 8); break;
            }
        }
#undef SPIKY_PROP
        return hipGetLastError();
    }
    const uint32_t n_ob = (s.n_outputs + s.ogs - 1) / s.ogs;
    const uint64_t n_items = (uint64_t)s.batch * s.n_detectors * n_ob;
    if (n_items == 0) return hipSuccess;
    if (int_mode)
        hipLaunchKernelGGL(k_propagate_fc_exact<true>, dim3(blocks_for(n_items)), dim3(kBlock), 0,
                           st, w, g, idx, min_deltas, min_idx, ap, x_grad, s.n_inputs,
                           s.n_outputs, s.n_detectors, s.n_anchors, s.n_entries, s.ogs, n_ob,
                           n_items, int_rescaler);
    else
        hipLaunchKernelGGL(k_propagate_fc_exact<false>, dim3(blocks_for(n_items)), dim3(kBlock),
                           0, st, w, g, idx, min_deltas, min_idx, ap, x_grad, s.n_inputs,
                           s.n_outputs, s.n_detectors, s.n_anchors, s.n_entries, s.ogs, n_ob,
                           n_items, int_rescaler);
    return hipGetLastError();
}

// scratch (bucketed path): bucket offsets [T][E+1] | sorted samples [T][B] |
// commit values [B][O]; the atomic fallback takes none
hipError_t launch_wgrad_fc(const FcShape &s, const float *g, const int32_t *idx, float *target,
                           double lr, bool int_mode, double int_rescaler, bool overwrite,
                           Scratch &scratch, hipStream_t st, const uint32_t *key_t,
                           uint32_t key_pitch, uint32_t key_shift) {
    const bool rowsum = rowsum_applies(s);
    ScratchLayout lay(scratch);
    int32_t *offsets = rowsum ? lay.take<int32_t>((size_t)s.n_detectors * (s.n_entries + 1) * 4) : nullptr;
    int32_t *samples = rowsum ? lay.take<int32_t>((size_t)s.n_detectors * s.batch * 4) : nullptr;
    uint32_t *cv = rowsum ? lay.take<uint32_t>((size_t)s.batch * s.n_outputs * 4) : nullptr;
    hipError_t e;
    if (lay.stop(&e, "gather_w_gradients_fc")) return e;
    if (rowsum) {
        e = launch_bucket_samples(s, idx, offsets, samples, st,
                                             s.n_entries <= 256 ? key_t : nullptr, key_pitch,
                                             key_shift);
        if (e != hipSuccess) return e;
        // 4 columns per lane once that still leaves 4 slices (two XCDs per slice)
        const uint32_t vec = (s.n_outputs % 4 == 0 && s.n_outputs >= 1024) ? 4 : pick_vec(s.n_outputs);
        const uint32_t n_slices = (s.n_outputs + kWave * vec - 1) / (kWave * vec);
        // rows a wavefront: 32, or fewer where few tables would leave the grid
        // short of 16 wavefronts a CU (a feed-forward layer's 16 tables)
        uint32_t rpw = std::min<uint32_t>(s.n_entries, 32);
        while (rpw > 4 && (uint64_t)n_slices * s.n_detectors * (s.n_entries / rpw) < 4096) rpw /= 2;
        const uint64_t units = (uint64_t)s.n_detectors * (s.n_entries / rpw);
        const uint64_t grid = (uint64_t)n_slices * ((units + kWPB - 1) / kWPB);
        if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
        const uint64_t n_cv = (uint64_t)s.batch * s.n_outputs;
        if (int_mode)
            hipLaunchKernelGGL(k_wgrad_commit_values<true>, dim3(blocks_for(n_cv)), dim3(kBlock), 0,
                               st, g, cv, n_cv, lr, int_rescaler);
        else
            hipLaunchKernelGGL(k_wgrad_commit_values<false>, dim3(blocks_for(n_cv)), dim3(kBlock), 0,
                               st, g, cv, n_cv, lr, int_rescaler);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
#define SPIKY_WG(V, IM, OW)                                                                       \
    hipLaunchKernelGGL((k_wgrad_slices<V, 8, IM, OW>), dim3((uint32_t)grid), dim3(kBlock), 0, st, \
                       cv, offsets, samples, target, s.batch, s.n_outputs, s.n_entries,           \
                       s.n_detectors, n_slices, rpw, int_rescaler)
#define SPIKY_WG_V(IM, OW)                     \
    switch (vec) {                             \
        case 4: SPIKY_WG(4, IM, OW); break;    \
        case 2: SPIKY_WG(2, IM, OW); break;    \
        default: SPIKY_WG(1, IM, OW); break;   \
    }
        if (int_mode) {
            if (overwrite) { SPIKY_WG_V(true, true) } else { SPIKY_WG_V(true, false) }
        } else {
            if (overwrite) { SPIKY_WG_V(false, true) } else { SPIKY_WG_V(false, false) }
        }
#undef SPIKY_WG_V
#undef SPIKY_WG
        return hipGetLastError();
    }
    // generic atomic fallback: the caller must have zeroed target when overwrite was asked for
    const uint64_t n_items = (uint64_t)s.batch * s.n_detectors * s.n_outputs;
    if (n_items == 0) return hipSuccess;
    if (overwrite) {
        e = launch_zero(target, (uint64_t)s.n_detectors * s.n_entries * s.n_outputs, st);
        if (e != hipSuccess) return e;
    }
    if (int_mode)
        hipLaunchKernelGGL(k_wgrad_fc_atomic<true>, dim3(blocks_for(n_items)), dim3(kBlock), 0, st,
                           g, idx, target, s.n_outputs, s.n_detectors, s.n_entries, n_items, lr,
                           int_rescaler);
    else
        hipLaunchKernelGGL(k_wgrad_fc_atomic<false>, dim3(blocks_for(n_items)), dim3(kBlock), 0,
                           st, g, idx, target, s.n_outputs, s.n_detectors, s.n_entries, n_items,
                           lr, int_rescaler);
    e = hipGetLastError();
    if (e != hipSuccess || !int_mode) return e;
    return launch_convert_i2f(target, (uint64_t)s.n_detectors * s.n_entries * s.n_outputs,
                              int_rescaler, st);
}

hipError_t launch_wgrad_commit_values(const float *g, uint32_t *cv, uint64_t n, double lr,
                                      bool int_mode, double int_rescaler, hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (int_mode)
        hipLaunchKernelGGL(k_wgrad_commit_values<true>, dim3(blocks_for(n)), dim3(kBlock), 0, st, g,
                           cv, n, lr, int_rescaler);
    else
        hipLaunchKernelGGL(k_wgrad_commit_values<false>, dim3(blocks_for(n)), dim3(kBlock), 0, st, g,
                           cv, n, lr, int_rescaler);
    return hipGetLastError();
}

hipError_t launch_bucket_samples(const FcShape &s, const int32_t *idx, int32_t *offsets,
                                 int32_t *samples, hipStream_t st, const uint32_t *key_t,
                                 uint32_t key_pitch, uint32_t key_shift) {
    if (s.n_detectors == 0) return hipSuccess;
    uint32_t n_bits = 0;
    while ((1u << n_bits) < s.n_entries) n_bits++;
    if (s.n_detectors < 1024 && s.batch >= 2048 && s.n_entries <= kBsMaxEntries) {
        // few tables over many samples: a workgroup per table
        hipLaunchKernelGGL(k_bucket_samples_wg, dim3(s.n_detectors), dim3(kBsThreads),
                           (size_t)kBsWaves * s.n_entries * sizeof(int32_t), st, idx, key_t, key_pitch,
                           key_shift, s.batch, s.n_detectors, s.n_entries, n_bits, offsets, samples);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_bucket_samples, dim3(s.n_detectors), dim3(kWave),
                       s.n_entries * sizeof(int32_t), st, idx, key_t, key_pitch, key_shift,
                       s.batch, s.n_detectors, s.n_entries, n_bits, offsets, samples);
    return hipGetLastError();
}

hipError_t launch_zero(float *buf, uint64_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_zero, dim3(blocks_for(n)), dim3(kBlock), 0, st, buf, n);
    return hipGetLastError();
}

hipError_t launch_convert_i2f(float *buf, uint64_t n, double int_rescaler, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_convert_i2f, dim3(blocks_for(n)), dim3(kBlock), 0, st, buf, n,
                       int_rescaler);
    return hipGetLastError();
}

}  // namespace spiky
