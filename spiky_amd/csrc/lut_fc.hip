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
//   k_check_detectors   one thread per (b, t).
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
struct RowLoad<int8_t, 4> {
    __device__ static void load(const int8_t *p, float *v) {
        const char4 q = *reinterpret_cast<const char4 *>(p);
        v[0] = (float)q.x;
        v[1] = (float)q.y;
        v[2] = (float)q.z;
        v[3] = (float)q.w;
    }
};

template <typename WT, int VEC, bool INT_MODE, bool SCALED, int DGS>
__global__ __launch_bounds__(kBlock) void k_fill_fc(
    const WT *__restrict__ w, const float *__restrict__ scales, const int32_t *__restrict__ idx,
    float *__restrict__ out, uint32_t batch, uint32_t n_outputs, uint32_t n_detectors,
    uint32_t n_entries, uint32_t dgs, uint32_t n_slices, double int_rescaler) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = uniform(threadIdx.x / kWave);
    const uint32_t slice = blockIdx.x % n_slices;
    const uint32_t b = (blockIdx.x / n_slices) * (kBlock / kWave) + wave;
    if (b >= batch) return;
    const uint32_t c = (slice * kWave + lane) * VEC;
    const bool active = c < n_outputs;
    const uint32_t emask = n_entries - 1;
    const int32_t *ib = idx + (size_t)b * n_detectors;
    float *ob = out + (size_t)b * n_outputs + c;

    float run[VEC];
    int32_t irun[VEC];
#pragma unroll
    for (int v = 0; v < VEC; v++) {
        run[v] = 0.0f;
        irun[v] = 0;
        if (active) {
            if (INT_MODE)
                irun[v] = __float_as_int(ob[v]);
            else
                run[v] = ob[v];
        }
    }

    const uint32_t block_len = DGS > 0 ? (uint32_t)DGS : dgs;
    for (uint32_t t0 = 0; t0 < n_detectors; t0 += block_len) {
        const uint32_t t1 = min(t0 + block_len, n_detectors);
        double acc[VEC];
#pragma unroll
        for (int v = 0; v < VEC; v++) acc[v] = 0.0;
        if (DGS > 0 && t1 - t0 == (uint32_t)DGS) {
            // full block: issue all DGS row loads before the ordered adds
            constexpr int kD = DGS > 0 ? DGS : 1;
            float vals[kD][VEC];
#pragma unroll
            for (int k = 0; k < kD; k++) {
                const uint32_t t = t0 + k;
                const uint32_t r = (uint32_t)ib[t] & emask;
                const WT *p = w + ((size_t)t * n_entries + r) * n_outputs + c;
                if (active) RowLoad<WT, VEC>::load(p, vals[k]);
                else {
#pragma unroll
                    for (int v = 0; v < VEC; v++) vals[k][v] = 0.0f;
                }
                if (SCALED) {
                    const float sc = scales[t];
#pragma unroll
                    for (int v = 0; v < VEC; v++) vals[k][v] = sc * vals[k][v];
                }
            }
#pragma unroll
            for (int k = 0; k < kD; k++) {
#pragma unroll
                for (int v = 0; v < VEC; v++) acc[v] += (double)vals[k][v];
            }
        } else {
#pragma unroll 8
            for (uint32_t t = t0; t < t1; t++) {
                const uint32_t r = (uint32_t)ib[t] & emask;
                const WT *p = w + ((size_t)t * n_entries + r) * n_outputs + c;
                float vals[VEC];
                if (active) RowLoad<WT, VEC>::load(p, vals);
                else {
#pragma unroll
                    for (int v = 0; v < VEC; v++) vals[v] = 0.0f;
                }
                if (SCALED) {
                    const float sc = scales[t];
#pragma unroll
                    for (int v = 0; v < VEC; v++) vals[v] = sc * vals[v];
                }
#pragma unroll
                for (int v = 0; v < VEC; v++) acc[v] += (double)vals[v];
            }
        }
#pragma unroll
        for (int v = 0; v < VEC; v++) {
            if (INT_MODE)
                irun[v] = wrap_add(irun[v], (int32_t)(acc[v] * kDenom32 * int_rescaler));
            else
                run[v] += (float)acc[v];
        }
    }
    if (!active) return;
#pragma unroll
    for (int v = 0; v < VEC; v++) {
        if (INT_MODE) {
            // convert_integers_to_floats_logic, proto:200-213
            const double y = (double)irun[v] * kDenom32Reciproc;
            ob[v] = (float)(y / int_rescaler);
        } else {
            ob[v] = run[v];
        }
    }
}

template <typename WT, int VEC, bool INT_MODE, bool SCALED>
hipError_t launch_fill_variant(const FcShape &s, const WT *w, const float *scales,
                               const int32_t *idx, float *out, double int_rescaler,
                               hipStream_t st) {
    const uint32_t cols_per_wave = kWave * VEC;
    const uint32_t n_slices = (s.n_outputs + cols_per_wave - 1) / cols_per_wave;
    const uint32_t waves_per_block = kBlock / kWave;
    const uint32_t b_groups = (s.batch + waves_per_block - 1) / waves_per_block;
    const uint64_t grid = (uint64_t)n_slices * b_groups;
    if (grid == 0) return hipSuccess;
    if (s.dgs == 32) {
        hipLaunchKernelGGL((k_fill_fc<WT, VEC, INT_MODE, SCALED, 32>), dim3((uint32_t)grid),
                           dim3(kBlock), 0, st, w, scales, idx, out, s.batch, s.n_outputs,
                           s.n_detectors, s.n_entries, s.dgs, n_slices, int_rescaler);
    } else {
        hipLaunchKernelGGL((k_fill_fc<WT, VEC, INT_MODE, SCALED, 0>), dim3((uint32_t)grid),
                           dim3(kBlock), 0, st, w, scales, idx, out, s.batch, s.n_outputs,
                           s.n_detectors, s.n_entries, s.dgs, n_slices, int_rescaler);
    }
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
// propagate, fast fp32-summation form: one wavefront per (sample, table chunk).
// Lane l owns columns (j*64 + l)*4 .. +3 for j < NJ.  The per-table result
// du * (sum_o W_main*g - sum_o W_alt*g) is reduced over the whole row in fp64
// and committed as one fp32 atomic pair per (b, t); the reference commits one
// pair per 32-output block, which differs only in fp32 rounding of the
// committed values (the blocks' du terms are summed in fp64 here first).
// ---------------------------------------------------------------------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <int NJ>
__global__ __launch_bounds__(kBlock) void k_propagate_fc_fast(
    const float *__restrict__ w, const float *__restrict__ g, const int32_t *__restrict__ idx,
    const float *__restrict__ md, const int32_t *__restrict__ mi, const int2 *__restrict__ anchors,
    float *__restrict__ x_grad, uint32_t batch, uint32_t n_inputs, uint32_t n_outputs,
    uint32_t n_detectors, uint32_t n_anchors, uint32_t n_entries, uint32_t n_chunks,
    uint32_t tables_per_chunk) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = uniform(threadIdx.x / kWave);
    const uint32_t chunk = blockIdx.x % n_chunks;
    const uint32_t b = (blockIdx.x / n_chunks) * (kBlock / kWave) + wave;
    if (b >= batch) return;
    const uint32_t t_begin = chunk * tables_per_chunk;
    const uint32_t t_end = min(t_begin + tables_per_chunk, n_detectors);
    const uint32_t emask = n_entries - 1;

    double gd[NJ][4];
    bool act[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const uint32_t c = (j * kWave + lane) * 4;
        act[j] = c < n_outputs;
        float4 gv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (act[j]) gv = *reinterpret_cast<const float4 *>(g + (size_t)b * n_outputs + c);
        gd[j][0] = gv.x;
        gd[j][1] = gv.y;
        gd[j][2] = gv.z;
        gd[j][3] = gv.w;
    }
    const int32_t *ib = idx + (size_t)b * n_detectors;
    const int32_t *mib = mi + (size_t)b * n_detectors;
    const float *mdb = md + (size_t)b * n_detectors;
    float *xg = x_grad + (size_t)b * n_inputs;

    for (uint32_t t = t_begin; t < t_end; t++) {
        const int32_t m = mib[t];
        const bool valid = m >= 0 && (uint32_t)m < n_anchors;
        const uint32_t r = (uint32_t)ib[t] & emask;
        const uint32_t ra = valid ? (r ^ (1u << m)) : r;
        const float *wm = w + ((size_t)t * n_entries + r) * n_outputs;
        const float *wa = w + ((size_t)t * n_entries + ra) * n_outputs;
        double dm = 0.0, da = 0.0;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (act[j]) {
                const uint32_t c = (j * kWave + lane) * 4;
                const float4 a = *reinterpret_cast<const float4 *>(wm + c);
                const float4 e = *reinterpret_cast<const float4 *>(wa + c);
                dm += (double)a.x * gd[j][0];
                dm += (double)a.y * gd[j][1];
                dm += (double)a.z * gd[j][2];
                dm += (double)a.w * gd[j][3];
                da += (double)e.x * gd[j][0];
                da += (double)e.y * gd[j][1];
                da += (double)e.z * gd[j][2];
                da += (double)e.w * gd[j][3];
            }
        }
        const double diff = wave_sum(dm - da);
        if (valid && lane == 0) {
            const double du = du_of_margin(mdb[t]) * diff;
            if (fabs(du) > kEps) {
                const int2 a = anchors[(size_t)t * n_anchors + m];
                if ((uint32_t)a.x < n_inputs && (uint32_t)a.y < n_inputs) {
                    unsafeAtomicAdd(xg + a.x, (float)du);
                    unsafeAtomicAdd(xg + a.y, (float)(-du));
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
__global__ __launch_bounds__(kWave) void k_bucket_samples(
    const int32_t *__restrict__ idx, uint32_t batch, uint32_t n_detectors, uint32_t n_entries,
    uint32_t n_bits, int32_t *__restrict__ offsets, int32_t *__restrict__ samples) {
    extern __shared__ int32_t cnt[];
    const uint32_t t = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const uint32_t emask = n_entries - 1;
    for (uint32_t e = lane; e < n_entries; e += kWave) cnt[e] = 0;
    __syncthreads();
    for (uint32_t base = 0; base < batch; base += kWave) {
        const uint32_t b = base + lane;
        if (b < batch) atomicAdd(&cnt[(uint32_t)idx[(size_t)b * n_detectors + t] & emask], 1);
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
    for (uint32_t base = 0; base < batch; base += kWave) {
        const uint32_t b = base + lane;
        const bool valid = b < batch;
        const uint32_t key = valid ? ((uint32_t)idx[(size_t)b * n_detectors + t] & emask) : 0u;
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
    }
}

// One wavefront per table row: target[row, :] (+)= sum over the row's bucket.
// Lane l owns columns (j*64 + l)*VEC .. +VEC-1 for j < NJ.
template <int NJ, int VEC, bool INT_MODE, bool OVERWRITE>
__global__ __launch_bounds__(kBlock) void k_wgrad_rowsum(
    const float *__restrict__ g, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ samples, float *__restrict__ target, uint32_t batch,
    uint32_t n_outputs, uint32_t n_entries, uint64_t n_rows, double lr, double int_rescaler) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint64_t wave0 = (uint64_t)blockIdx.x * (kBlock / kWave) + uniform(threadIdx.x / kWave);
    const uint64_t n_waves = (uint64_t)gridDim.x * (kBlock / kWave);
    for (uint64_t row = wave0; row < n_rows; row += n_waves) {
        const uint32_t t = (uint32_t)(row / n_entries);
        const uint32_t e = (uint32_t)(row % n_entries);
        const int32_t *off_t = offsets + (size_t)t * (n_entries + 1);
        const int32_t beg = off_t[e];
        const int32_t end = off_t[e + 1];
        if (!OVERWRITE && !INT_MODE && beg == end) continue;
        const int32_t *smp = samples + (size_t)t * batch;
        float *trow = target + row * n_outputs;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t c = (j * kWave + lane) * VEC;
            if (c >= n_outputs) continue;
            float acc[VEC];
            int32_t iacc[VEC];
#pragma unroll
            for (int q = 0; q < VEC; q++) {
                acc[q] = 0.0f;
                iacc[q] = 0;
            }
            if (!OVERWRITE) {
                float v[VEC];
                RowLoad<float, VEC>::load(trow + c, v);
#pragma unroll
                for (int q = 0; q < VEC; q++) {
                    acc[q] = v[q];
                    iacc[q] = __float_as_int(v[q]);
                }
            }
            for (int32_t k = beg; k < end; k++) {
                const uint32_t b = (uint32_t)smp[k];
                float gs[VEC];
                RowLoad<float, VEC>::load(g + (size_t)b * n_outputs + c, gs);
#pragma unroll
                for (int q = 0; q < VEC; q++) {
                    const double gg = (double)gs[q];
                    if (fabs(gg) > kEps) {
                        if (INT_MODE)
                            iacc[q] = wrap_add(iacc[q], (int32_t)(gg * lr * kDenom32 * int_rescaler));
                        else
                            acc[q] += (float)(gg * lr);
                    }
                }
            }
            float res[VEC];
#pragma unroll
            for (int q = 0; q < VEC; q++)
                res[q] = INT_MODE ? (float)(((double)iacc[q] * kDenom32Reciproc) / int_rescaler) : acc[q];
            if (VEC == 4)
                *reinterpret_cast<float4 *>(trow + c) = make_float4(res[0], res[1], res[2], res[3]);
            else
#pragma unroll
                for (int q = 0; q < VEC; q++) trow[c + q] = res[q];
        }
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

bool rowsum_applies(const FcShape &s) {
    const uint32_t vec = (s.n_outputs % 4 == 0) ? 4 : 1;
    return s.n_outputs <= 16u * 64u * vec && s.n_entries <= 4096 && s.batch <= 0x7fffffffu;
}

}  // namespace

// ---------------------------------------------------------------------------
hipError_t launch_check_detectors(const FcShape &s, const float *x, const int32_t *anchors,
                                  float cmp_eps, int32_t *idx, float *min_deltas,
                                  int32_t *min_idx, hipStream_t st) {
    const uint32_t bpr = (s.n_detectors + kBlock - 1) / kBlock;
    const uint64_t grid = (uint64_t)bpr * s.batch;
    if (grid == 0) return hipSuccess;
    const int2 *ap = reinterpret_cast<const int2 *>(anchors);
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
    if (s.n_outputs % 2 == 0) {
        if (int_mode)
            return launch_fill_variant<float, 2, true, false>(s, w, nullptr, idx, out,
                                                              int_rescaler, st);
        return launch_fill_variant<float, 2, false, false>(s, w, nullptr, idx, out, int_rescaler,
                                                           st);
    }
    if (int_mode)
        return launch_fill_variant<float, 1, true, false>(s, w, nullptr, idx, out, int_rescaler,
                                                          st);
    return launch_fill_variant<float, 1, false, false>(s, w, nullptr, idx, out, int_rescaler, st);
}

hipError_t launch_fill_fc_i8(const FcShape &s, const int8_t *q8, const float *scales,
                             const int32_t *idx, float *out, bool int_mode, double int_rescaler,
                             hipStream_t st) {
    if (s.n_outputs % 4 == 0) {
        if (int_mode)
            return launch_fill_variant<int8_t, 4, true, true>(s, q8, scales, idx, out,
                                                              int_rescaler, st);
        return launch_fill_variant<int8_t, 4, false, true>(s, q8, scales, idx, out, int_rescaler,
                                                           st);
    }
    if (int_mode)
        return launch_fill_variant<int8_t, 1, true, true>(s, q8, scales, idx, out, int_rescaler,
                                                          st);
    return launch_fill_variant<int8_t, 1, false, true>(s, q8, scales, idx, out, int_rescaler, st);
}

hipError_t launch_propagate_fc(const FcShape &s, const float *w, const float *g,
                               const int32_t *idx, const float *min_deltas,
                               const int32_t *min_idx, const int32_t *anchors, float *x_grad,
                               bool int_mode, double int_rescaler, hipStream_t st) {
    const int2 *ap = reinterpret_cast<const int2 *>(anchors);
    const uint32_t nj = (s.n_outputs + 255) / 256;
    const bool fast = !int_mode && s.n_outputs % 4 == 0 && nj <= 4 && s.n_detectors >= 64;
    if (fast) {
        const uint32_t n_chunks = std::min<uint32_t>(8, s.n_detectors);
        const uint32_t tpc = (s.n_detectors + n_chunks - 1) / n_chunks;
        const uint32_t b_groups = (s.batch + 3) / 4;
        const uint64_t grid = (uint64_t)n_chunks * b_groups;
#define SPIKY_PROP_FAST(NJ)                                                                      \
    hipLaunchKernelGGL(k_propagate_fc_fast<NJ>, dim3((uint32_t)grid), dim3(kBlock), 0, st, w, g, \
                       idx, min_deltas, min_idx, ap, x_grad, s.batch, s.n_inputs, s.n_outputs,  \
                       s.n_detectors, s.n_anchors, s.n_entries, n_chunks, tpc)
        switch (nj) {
            case 1: SPIKY_PROP_FAST(1); break;
            case 2: SPIKY_PROP_FAST(2); break;
            case 3: SPIKY_PROP_FAST(3); break;
            default: SPIKY_PROP_FAST(4); break;
        }
#undef SPIKY_PROP_FAST
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

size_t wgrad_fc_scratch_bytes(const FcShape &s) {
    if (!rowsum_applies(s)) return 0;
    return ((size_t)s.n_detectors * (s.n_entries + 1) + (size_t)s.n_detectors * s.batch) *
           sizeof(int32_t);
}

hipError_t launch_wgrad_fc(const FcShape &s, const float *g, const int32_t *idx, float *target,
                           double lr, bool int_mode, double int_rescaler, bool overwrite,
                           void *scratch, hipStream_t st) {
    if (rowsum_applies(s) && scratch != nullptr) {
        int32_t *offsets = reinterpret_cast<int32_t *>(scratch);
        int32_t *samples = offsets + (size_t)s.n_detectors * (s.n_entries + 1);
        hipError_t e = launch_bucket_samples(s, idx, offsets, samples, st);
        if (e != hipSuccess) return e;
        const uint64_t n_rows = (uint64_t)s.n_detectors * s.n_entries;
        const uint64_t want = (n_rows + 3) / 4;
        const uint32_t grid = (uint32_t)std::min<uint64_t>(want, 65536);
        const uint32_t vec = (s.n_outputs % 4 == 0) ? 4 : 1;
        const uint32_t nj = (s.n_outputs + 64 * vec - 1) / (64 * vec);
#define SPIKY_ROWSUM(NJ, V, IM, OW)                                                               \
    hipLaunchKernelGGL((k_wgrad_rowsum<NJ, V, IM, OW>), dim3(grid), dim3(kBlock), 0, st, g,        \
                       offsets, samples, target, s.batch, s.n_outputs, s.n_entries, n_rows, lr,  \
                       int_rescaler)
#define SPIKY_ROWSUM_NJ(IM, OW)                                          \
    if (vec == 4) {                                                      \
        switch (nj) {                                                    \
            case 1: SPIKY_ROWSUM(1, 4, IM, OW); break;                   \
            case 2: SPIKY_ROWSUM(2, 4, IM, OW); break;                   \
            case 3: SPIKY_ROWSUM(3, 4, IM, OW); break;                   \
            case 4: SPIKY_ROWSUM(4, 4, IM, OW); break;                   \
            case 5: case 6: case 7: case 8: SPIKY_ROWSUM(8, 4, IM, OW); break; \
            default: SPIKY_ROWSUM(16, 4, IM, OW); break;                 \
        }                                                                \
    } else {                                                             \
        switch (nj) {                                                    \
            case 1: SPIKY_ROWSUM(1, 1, IM, OW); break;                   \
            case 2: SPIKY_ROWSUM(2, 1, IM, OW); break;                   \
            case 3: case 4: SPIKY_ROWSUM(4, 1, IM, OW); break;           \
            case 5: case 6: case 7: case 8: SPIKY_ROWSUM(8, 1, IM, OW); break; \
            default: SPIKY_ROWSUM(16, 1, IM, OW); break;                 \
        }                                                                \
    }
        if (int_mode) {
            if (overwrite) { SPIKY_ROWSUM_NJ(true, true) } else { SPIKY_ROWSUM_NJ(true, false) }
        } else {
            if (overwrite) { SPIKY_ROWSUM_NJ(false, true) } else { SPIKY_ROWSUM_NJ(false, false) }
        }
#undef SPIKY_ROWSUM_NJ
#undef SPIKY_ROWSUM
        return hipGetLastError();
    }
    // generic atomic fallback: the caller must have zeroed target when overwrite was asked for
    const uint64_t n_items = (uint64_t)s.batch * s.n_detectors * s.n_outputs;
    if (n_items == 0) return hipSuccess;
    if (overwrite) {
        hipError_t e = launch_zero(target, (uint64_t)s.n_detectors * s.n_entries * s.n_outputs, st);
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
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !int_mode) return e;
    return launch_convert_i2f(target, (uint64_t)s.n_detectors * s.n_entries * s.n_outputs,
                              int_rescaler, st);
}

hipError_t launch_bucket_samples(const FcShape &s, const int32_t *idx, int32_t *offsets,
                                 int32_t *samples, hipStream_t st) {
    if (s.n_detectors == 0) return hipSuccess;
    uint32_t n_bits = 0;
    while ((1u << n_bits) < s.n_entries) n_bits++;
    hipLaunchKernelGGL(k_bucket_samples, dim3(s.n_detectors), dim3(kWave),
                       s.n_entries * sizeof(int32_t), st, idx, s.batch, s.n_detectors,
                       s.n_entries, n_bits, offsets, samples);
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
