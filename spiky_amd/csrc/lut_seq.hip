// lut_seq.hip -- sequence-concat LUT kernels (LUTTransformer attention) for gfx950.
//
// Layouts (caller-owned, as in the reference): x [B][S][I]; idx / md / mi
// [B][S][T]; positional embeddings [(S-1)][T][Npe]; pidx / pmd / pmi
// [(S-1)][T]; out / g [B][S][O]; W [T][2^(2Nc+Npe)][O] with row
// (Q << (Nc+Npe)) | (K << Npe) | PE, where Q is the later position's index,
// K the earlier one's and PE the index of their distance - 1
// (lut_runtime_kernels_logic.proto:1807-1904, lut.cu:42).
//
// Kernels:
//   k_check_pe          one thread per (distance, table): sign bits of the
//                       positional embedding and its min-|value| dimension.
//   k_seq_pack          idx / mi / md -> one 8-byte record per (t, b, s), so a
//                       wavefront's walk over positions reads contiguous memory.
//   k_fill_seq          one wavefront per (sample, later position j, column
//                       slice): tables in ascending order, pairs i < j summed in
//                       fp64 and committed once per table -- the reference CPU
//                       path's order, so the output is bit-identical to it.
//   k_propagate_seq     fp32 summation: one wavefront per (sample, table, j); for
//                       8 pairs at a time it reads the main, flipped and
//                       PE-flipped rows, reduces the dots with a DPP
//                       reduce-scatter, keeps the Q-flip terms of (b, t, j) in
//                       registers and adds K-flip and positional terms with fp64
//                       atomics into small per-(b, t, position) buffers.
//   k_propagate_seq_exact  int32 summation (and any shape): the reference's own
//                       decomposition, one thread per (pair, table, output block)
//                       with sequential block dots and integer payloads, so the
//                       int32 accumulators are bit-identical.
//   k_seq_xgrad         x_grad[b][s][anchor] +-= du(b, t, s) for every table.
//   k_wgrad_seq_sort    one workgroup per (table, Q value): an LDS counting sort
//                       of the (b, j, i) entries of every (b, j) whose Q is that
//                       value by target row, then per column slice the
//                       sub-table's gradient (2^(Nc+Npe) rows x C columns) is
//                       summed in registers and written once.
#include "lut_kernels.h"

#include <algorithm>
#include <type_traits>
#include <utility>

namespace spiky {
namespace {

constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWPB = kBlock / kWave;

__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
// lane l's value of v (a scalar read, the same in every lane)
__device__ __forceinline__ double readlane_f64(double v, int l) {
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

__device__ __forceinline__ bool rounded_greater0(float d, float cmp_eps) {
    if (cmp_eps == 0.0f) return d > 0.0f;
    return (fabsf(d) < cmp_eps) ? false : (d > 0.0f);
}

__device__ __forceinline__ double du_of_margin(float md) {
    double du = (double)md;
    double r = 1.0 / (1.0 + fabs(du));
    return (du > 0) ? r * (0.5 * r) : r * (-0.5 * r);
}

// DPP lane exchange of an fp64 value.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)(uint32_t)hi << 32) |
                                            (unsigned long long)(uint32_t)lo));
}

// Record of one (table, sample, position): x = md bits, y = idx | (mi & 0xff) << 16.
__device__ __forceinline__ uint32_t rec_idx(uint2 r) { return r.y & 0xFFFFu; }
__device__ __forceinline__ int32_t rec_mi(uint2 r) {
    const uint32_t m = (r.y >> 16) & 0xFFu;
    return m == 0xFFu ? -1 : (int32_t)m;
}
__device__ __forceinline__ float rec_md(uint2 r) { return __uint_as_float(r.x); }

// ---------------------------------------------------------------------------
// check_positional_embeddings(_eval)_logic, proto:1709-1805
template <bool TRAIN>
__global__ __launch_bounds__(kBlock) void k_check_pe(const float *__restrict__ pe, uint32_t n_items,
                                                     uint32_t pe_dim, float cmp_eps,
                                                     int32_t *__restrict__ pidx,
                                                     float *__restrict__ pmd,
                                                     int32_t *__restrict__ pmi) {
    const uint32_t it = blockIdx.x * kBlock + threadIdx.x;
    if (it >= n_items) return;
    const float *v = pe + (size_t)it * pe_dim;
    int32_t li = 0, mk = -1;
    float mind = 0.0f;
    for (uint32_t d = 0; d < pe_dim; d++) {
        const float x = v[d];
        if (rounded_greater0(x, cmp_eps)) li |= (1 << d);
        if (TRAIN && (mk == -1 || fabsf(x) < fabsf(mind))) {
            mind = x;
            mk = (int32_t)d;
        }
    }
    pidx[it] = li;
    if (TRAIN) {
        pmd[it] = mind;
        pmi[it] = mk;
    }
}

// pack[t][b][s] from idx / md / mi [b][s][t] (md / mi may be null: eval).
__global__ __launch_bounds__(kBlock) void k_seq_pack(const int32_t *__restrict__ idx,
                                                     const float *__restrict__ md,
                                                     const int32_t *__restrict__ mi,
                                                     uint2 *__restrict__ pack, uint32_t n_rows,
                                                     uint32_t n_detectors) {
    __shared__ uint2 tile[64][65];
    const uint32_t tb = blockIdx.x * 64;  // tables
    const uint32_t rb = blockIdx.y * 64;  // rows b*S + s
    const uint32_t tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t row = rb + r, t = tb + tx;
        if (row < n_rows && t < n_detectors) {
            const size_t o = (size_t)row * n_detectors + t;
            const uint32_t m = mi ? (uint32_t)(mi[o] < 0 ? 0xFF : mi[o] & 0xFF) : 0xFFu;
            tile[r][tx] = make_uint2(md ? __float_as_uint(md[o]) : 0u,
                                     ((uint32_t)idx[o] & 0xFFFFu) | (m << 16));
        }
    }
    __syncthreads();
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t t = tb + r, row = rb + tx;
        if (row < n_rows && t < n_detectors) pack[(size_t)t * n_rows + row] = tile[tx][r];
    }
}

// ppack[t][d] from pidx / pmd / pmi [d][t]; all zero (PE index 0) without PE.
__global__ __launch_bounds__(kBlock) void k_seq_pack_pe(const int32_t *__restrict__ pidx,
                                                        const float *__restrict__ pmd,
                                                        const int32_t *__restrict__ pmi,
                                                        uint2 *__restrict__ ppack, uint32_t n_dist,
                                                        uint32_t n_detectors) {
    const uint32_t it = blockIdx.x * kBlock + threadIdx.x;
    if (it >= n_dist * n_detectors) return;
    const uint32_t t = it / n_dist, d = it % n_dist;
    uint2 r = make_uint2(0u, 0xFFu << 16);
    if (pidx) {
        const size_t o = (size_t)d * n_detectors + t;
        const uint32_t m = pmi ? (uint32_t)(pmi[o] < 0 ? 0xFF : pmi[o] & 0xFF) : 0xFFu;
        r = make_uint2(pmd ? __float_as_uint(pmd[o]) : 0u, ((uint32_t)pidx[o] & 0xFFFFu) | (m << 16));
    }
    ppack[it] = r;
}

// ---------------------------------------------------------------------------
// fill_outputs_fully_connected_seq_logic (proto:1807-1904), re-scheduled.
template <int VEC>
struct Ld;
template <>
struct Ld<1> {
    __device__ static void f(const float *p, float *v) { v[0] = p[0]; }
};
template <>
struct Ld<2> {
    __device__ static void f(const float *p, float *v) {
        const float2 q = *reinterpret_cast<const float2 *>(p);
        v[0] = q.x;
        v[1] = q.y;
    }
};
template <>
struct Ld<4> {
    __device__ static void f(const float *p, float *v) {
        const float4 q = *reinterpret_cast<const float4 *>(p);
        v[0] = q.x;
        v[1] = q.y;
        v[2] = q.z;
        v[3] = q.w;
    }
};

template <int VEC, bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_fill_seq(
    const float *__restrict__ w, const uint2 *__restrict__ pack, const uint2 *__restrict__ ppack,
    float *__restrict__ out, uint32_t batch, uint32_t seq, uint32_t n_outputs,
    uint32_t n_detectors, uint32_t n_anchors, uint32_t pe_dim, uint32_t n_slices,
    double int_rescaler) {
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = uniform(threadIdx.x / kWave);
    const uint32_t slice = blockIdx.x % n_slices;
    const uint32_t unit = (blockIdx.x / n_slices) * kWPB + wave;
    const uint32_t per_b = seq - 1;
    const uint32_t b = unit / per_b;
    if (b >= batch) return;
    const uint32_t j = seq - 1 - unit % per_b;  // long rows first
    const uint32_t c = (slice * kWave + lane) * VEC;
    const bool active = c < n_outputs;
    const uint32_t cc = active ? c : 0u;
    const uint32_t n_rows = batch * seq;
    const uint32_t sub_rows = 1u << (n_anchors + pe_dim);  // rows per (table, Q)
    float *ob = out + ((size_t)b * seq + j) * n_outputs + c;
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
    for (uint32_t t = 0; t < n_detectors; t++) {
        const uint2 *kp = pack + (size_t)t * n_rows + (size_t)b * seq;
        const uint2 *pp = ppack + (size_t)t * (seq - 1);
        const uint32_t q = rec_idx(kp[j]);
        const float *sub = w + ((size_t)t * (1u << n_anchors) + q) * sub_rows * n_outputs + cc;
        double acc[VEC];
#pragma unroll
        for (int v = 0; v < VEC; v++) acc[v] = 0.0;
        for (uint32_t i0 = 0; i0 < j; i0 += 8) {
            const uint32_t n = min(8u, j - i0);
            float vals[8][VEC];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t i = i0 + min((uint32_t)u, n - 1);
                const uint32_t row = (rec_idx(kp[i]) << pe_dim) | rec_idx(pp[j - i - 1]);
                Ld<VEC>::f(sub + (size_t)(row & (sub_rows - 1)) * n_outputs, vals[u]);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if ((uint32_t)u < n) {
#pragma unroll
                    for (int v = 0; v < VEC; v++) acc[v] += (double)vals[u][v];
                }
            }
        }
        if (j == 0) continue;
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
    for (int v = 0; v < VEC; v++)
        ob[v] = INT_MODE ? (float)(((double)irun[v] * kDenom32Reciproc) / int_rescaler) : run[v];
}

// ---------------------------------------------------------------------------
// Sub-table-major forward: one 1024-thread workgroup per (table t, Q value q,
// column slice of C columns).  The sub-table slice W[t][q][*][c0, c0 + C)
// (2^(Nc+Npe) rows, at most 128 KiB) is staged in LDS once, so each table byte
// crosses HBM once per forward.  The items (b, j) of the bucket (t, q) are
// taken longest-first (an LDS counting sort on length classes); C lanes own one item and sum
// its pairs i < j in ascending i in fp64, reading rows from LDS.  The commit
// value of table t, fp32(sum) (int mode: the int32 payload), goes to
// part[t][b*S + j][o]; k_fill_commit adds the tables in ascending order, the
// reference CPU path's order (proto:1807-1904), so the output is bit-identical.
// Position 0 has no pairs: its value is -0.0f (0 in int mode), which leaves
// every sum unchanged.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// A workgroup barrier that orders LDS only: this wave's LDS accesses are complete
// before it, while its vector-memory loads (an LDS DMA) may still be in flight.
// __syncthreads' fence would wait for those as well.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// LDS byte address of a __shared__ location
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p;
}
// A 16-byte LDS DMA per lane: global g -> LDS byte address lds + 16 * lane (lds
// is the wavefront's base).  Issued as an instruction the compiler does not see
// into: with the builtin, every later LDS access of the kernel waits for the
// DMA, since the compiler cannot tell the destination apart from the other LDS
// arrays.  The caller waits for it with an explicit vmcnt before reading the
// destination.  M0 is restored, so the compiler's own use of it is unaffected.
// For a load issued before it and used after it, the compiler's vmcnt wait
// counts too few loads behind that one: the wait is only stricter (in order).
__device__ __forceinline__ void dma16_unseen(const void *g, uint32_t lds) {
    const uint32_t a = __builtin_amdgcn_readfirstlane(lds);
    uint32_t keep;
    __asm__ volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(keep)
        : "s"(a), "v"(g)
        : "memory");
}

constexpr int kSfThreads = 1024;
constexpr int kSfTabFloats = 32768;   // 128 KiB sub-table slice
constexpr int kSfItems = 1024;        // items sorted per chunk of a bucket
static_assert(kSfItems % kSfThreads == 0, "whole item rows per thread");
constexpr int kSfPe = 2048;           // distances S - 1
constexpr int kSfLenClasses = 256;    // item length classes of the longest-first order

// VW consecutive columns of one LDS row (VW = 1, 2 or 4 floats).
template <int VW>
__device__ __forceinline__ void lds_cols(const uint8_t *p, float (&v)[VW]) {
    if constexpr (VW == 4) {
        const f32x4 q = *reinterpret_cast<const f32x4 *>(p);
        v[0] = q[0]; v[1] = q[1]; v[2] = q[2]; v[3] = q[3];
    } else if constexpr (VW == 2) {
        const float2 q = *reinterpret_cast<const float2 *>(p);
        v[0] = q.x; v[1] = q.y;
    } else {
        v[0] = *reinterpret_cast<const float *>(p);
    }
}

// v from lane M of this lane's 16-lane row (DPP row_newbcast); folded into the
// add that uses it
template <int M>
__device__ __forceinline__ uint32_t row_bcast(uint32_t v) {
    return __builtin_amdgcn_update_dpp(0u, v, 0x150 + M, 0xF, 0xF, false);
}

// Pairs of a chunk of 16 n pairs whose LDS row offsets lie one per lane of the
// item's 16-lane row (pair M in lane M % 16, register M / 16): sixteen pairs'
// VW columns read (all in flight), then added to the fp64 sums in ascending M.
template <int M>
struct SeqPairs16 {
    template <int VW, int KP>
    __device__ __forceinline__ static void read(const uint8_t *tb, const uint32_t (&off)[KP], float (&v)[16][VW]) {
        SeqPairs16<M - 1>::template read<VW, KP>(tb, off, v);
        lds_cols<VW>(tb + row_bcast<(M - 1) % 16>(off[(M - 1) / 16]), v[(M - 1) % 16]);
    }
};
template <>
struct SeqPairs16<0> {
    template <int VW, int KP>
    __device__ __forceinline__ static void read(const uint8_t *, const uint32_t (&)[KP], float (&)[16][VW]) {}
};
template <int VW, int KP, int M0>
__device__ __forceinline__ void seq_group_add(const uint8_t *tb, const uint32_t (&off)[KP], double (&acc)[VW]) {
    float v[16][VW];
    // offsets of pairs M0 .. M0 + 15: register M0 / 16, lanes 0 .. 15
    const uint32_t (&o)[KP] = off;
    uint32_t one[1] = {o[M0 / 16]};
    SeqPairs16<16>::template read<VW, 1>(tb, one, v);
#pragma unroll
    for (int m = 0; m < 16; m++)
#pragma unroll
        for (int c = 0; c < VW; c++) acc[c] += (double)v[m][c];  // ascending pairs: ascending i
}
template <int VW, int KP, int... Gs>
__device__ __forceinline__ void seq_chunk_add(const uint8_t *tb, const uint32_t (&off)[KP], double (&acc)[VW],
                                              std::integer_sequence<int, Gs...>) {
    (seq_group_add<VW, KP, 16 * Gs>(tb, off, acc), ...);
}

// C / VW lanes own an item, lane l of it holding columns VW l .. VW l + VW-1 of
// the slice (VW = 4 at 64-column slices, 2 at 32, 1 below): 16 lanes an item,
// so a bucket of ~128 items makes ~32 item groups for the 16 wavefronts and
// the longest-first queue balances them; one VW-float LDS read per pair and
// VW independent fp64 sums, each taking the pairs in ascending i.
template <int C, bool INT_MODE>
__global__ __launch_bounds__(kSfThreads) void k_fill_seq_lds(
    const float *__restrict__ w, const uint2 *__restrict__ pack, const uint2 *__restrict__ ppack,
    const int32_t *__restrict__ offsets, const int32_t *__restrict__ samples,
    const uint32_t *__restrict__ order, uint32_t *__restrict__ part, uint32_t batch, uint32_t seq,
    uint32_t n_outputs, uint32_t n_anchors, uint32_t pe_dim, uint32_t n_slices, double int_rescaler) {
    constexpr int VW = C >= 64 ? 4 : (C >= 32 ? 2 : 1);  // columns per lane
    constexpr int L = C / VW;          // lanes per item
    constexpr int kSlots = kWave / L;  // items per wavefront
    constexpr int kPer = C / L;        // row offsets each lane forms per chunk of C pairs (VW)
    __shared__ __attribute__((aligned(16))) float tab[kSfTabFloats + 64];  // + a zero row
    __shared__ __attribute__((aligned(16))) uint32_t rowtab[(kSfThreads / kWave) * kSlots * C];
    __shared__ uint16_t ptab[kSfPe];
    __shared__ uint32_t keys[kSfItems];
    __shared__ uint32_t irow[kSfItems];
    __shared__ uint32_t jhist[kSfLenClasses];
    __shared__ uint32_t next_item;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = tid / kWave;
    uint32_t jsh = 0;  // length classes: (S - 1 - j) >> jsh < kSfLenClasses
    while (((seq - 1) >> jsh) >= (uint32_t)kSfLenClasses) jsh++;
    const uint32_t half = lane / L, cl = lane % L;
    uint32_t *my_rows = rowtab + (wave * kSlots + half) * C;
    const uint32_t slice = blockIdx.x % n_slices;
    const uint32_t tq = order ? order[blockIdx.x / n_slices] : blockIdx.x / n_slices;  // largest first
    const uint32_t n_q = 1u << n_anchors;
    const uint32_t t = tq / n_q, q = tq % n_q;
    const uint32_t sub_rows = 1u << (n_anchors + pe_dim);
    const uint32_t pmask = (1u << pe_dim) - 1;
    const uint32_t n_rows = batch * seq;
    const uint32_t c0 = slice * C;
    const int32_t beg = offsets[(size_t)t * (n_q + 1) + q];
    const int32_t end = offsets[(size_t)t * (n_q + 1) + q + 1];
    if (beg >= end) return;  // uniform over the workgroup

    const int32_t *smp = samples + (size_t)t * n_rows;
    const uint2 *kp = pack + (size_t)t * n_rows;
    const uint32_t col = c0 + cl * VW;
    const float *sub = w + ((size_t)t * n_q + q) * sub_rows * n_outputs + c0;
    const uint32_t n_e = sub_rows * (C / 4);
    const uint32_t zero_off = sub_rows * C * 4;  // byte offset of the zero row
    const uint8_t *tab_b = reinterpret_cast<const uint8_t *>(tab) + cl * VW * 4;

    // the first chunk's item rows: loads in flight with the staging loads
    uint32_t rr[kSfItems / kSfThreads];
#pragma unroll
    for (int u = 0; u < kSfItems / kSfThreads; u++) {
        const uint32_t it = u * kSfThreads + tid;
        rr[u] = (int32_t)it < end - beg ? (uint32_t)smp[beg + it] : 0u;
    }
    // the positional indices first: their loads are waited for before the
    // table's are issued
    for (uint32_t d = tid; d + 1 < seq; d += kSfThreads)
        ptab[d] = (uint16_t)(rec_idx(ppack[(size_t)t * (seq - 1) + d]) & pmask);
    if (tid < (uint32_t)C) tab[sub_rows * C + tid] = 0.0f;
    // the first chunk's item rows, in LDS before the table's loads are issued
    // (stored by every lane, 0 past the chunk's end: no load is left pending
    // on any path, which would make the compiler wait for the DMA as well)
#pragma unroll
    for (int u = 0; u < kSfItems / kSfThreads; u++) irow[u * kSfThreads + tid] = rr[u];
    // stage the slice: C / 4 lanes per row, 16-byte pieces (O % 4 == 0), piece e
    // at byte 16 e of the [row][C] image.  A slice inside the row goes by LDS DMA,
    // so the first chunk's counting sort runs while it lands (the walk waits for
    // it); a slice past the row's end, through registers with zeros past it.
    const bool slice_dma = c0 + C <= n_outputs;  // uniform
    if (slice_dma) {
        const uint32_t tab_lds = lds_addr(tab);
        for (uint32_t e0 = 0; e0 < n_e; e0 += kSfThreads) {
            const uint32_t e = e0 + tid;
            if (e < n_e) {
                const uint32_t r = e / (C / 4), c4 = (e % (C / 4)) * 4;
                dma16_unseen(sub + (size_t)r * n_outputs + c4, tab_lds + (e0 + wave * kWave) * 16);
            }
        }
    } else {
        for (uint32_t e0 = 0; e0 < n_e; e0 += 8 * kSfThreads) {
            f32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t e = e0 + u * kSfThreads + tid;
                const uint32_t r = e / (C / 4), c4 = (e % (C / 4)) * 4;
                v[u] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (e < n_e && c0 + c4 < n_outputs)
                    v[u] = *reinterpret_cast<const f32x4 *>(sub + (size_t)r * n_outputs + c4);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t e = e0 + u * kSfThreads + tid;
                if (e < n_e) *reinterpret_cast<f32x4 *>(tab + (e / (C / 4)) * C + (e % (C / 4)) * 4) = v[u];
            }
        }
        // vmcnt(0), as the compiler's own wait: no load of this branch stays
        // pending where it joins the DMA branch
        __builtin_amdgcn_s_waitcnt(0xF70);
    }

    // key record words of positions i (.y words)
    const uint32_t *kw = reinterpret_cast<const uint32_t *>(kp) + 1;
    // One chunk of the bucket's items, whose rows are in irow: the longest-first
    // sort and the walk.  The first chunk runs outside the loop that loads the
    // later chunks' rows, so nothing but the table DMA is in flight before the
    // walk's wait for it, and the sort overlaps the DMA.
    auto run_chunk = [&](int32_t k0, uint32_t n) {
        lds_barrier();  // the chunk's item rows in irow
        // Longest first: a counting sort of the items on (S - 1 - j) >> jsh (at most
        // kSfLenClasses classes; the order within a class is arbitrary), keys[pos]
        // = the item's number in the chunk.
        for (uint32_t k = tid; k < (uint32_t)kSfLenClasses; k += kSfThreads) jhist[k] = 0;
        lds_barrier();
        uint32_t cls[kSfItems / kSfThreads], rank[kSfItems / kSfThreads];
#pragma unroll
        for (int u = 0; u < kSfItems / kSfThreads; u++) {
            const uint32_t it = u * kSfThreads + tid;
            if (it < n) {
                cls[u] = (seq - 1 - irow[it] % seq) >> jsh;
                rank[u] = atomicAdd(&jhist[cls[u]], 1u);
            }
        }
        lds_barrier();
        if (wave == 0) {  // exclusive scan of the class counts
            constexpr int kPerLane = kSfLenClasses / kWave;
            uint32_t c[kPerLane], sum = 0;
#pragma unroll
            for (int k = 0; k < kPerLane; k++) {
                c[k] = jhist[lane * kPerLane + k];
                sum += c[k];
            }
            uint32_t inc = sum;
#pragma unroll
            for (int o = 1; o < kWave; o <<= 1) {
                const uint32_t y = __shfl_up(inc, o, kWave);
                if (lane >= (uint32_t)o) inc += y;
            }
            uint32_t run = inc - sum;
#pragma unroll
            for (int k = 0; k < kPerLane; k++) {
                jhist[lane * kPerLane + k] = run;
                run += c[k];
            }
        }
        lds_barrier();
#pragma unroll
        for (int u = 0; u < kSfItems / kSfThreads; u++) {
            const uint32_t it = u * kSfThreads + tid;
            if (it < n) keys[jhist[cls[u]] + rank[u]] = it;
        }
        if (tid == 0) next_item = 0;
        // the table slice has landed (this wave's DMA; the barrier, everyone's)
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // items are taken kSlots at a time, longest first; the next group's rows
        // and first key records are fetched while the current group runs
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(&next_item, (uint32_t)kSlots);
        base = uniform(__shfl(base, 0, kWave));
        uint32_t my = base + half;
        bool have = my < n;
        uint32_t row = have ? irow[keys[my] & 0xFFFFu] : 0u;
        uint32_t j = have ? row % seq : 0u;
        // key records of this lane's pairs of a chunk (i = i0 + cl + L k),
        // loaded unconditionally (index clamped into the sample) one chunk
        // ahead, and first read through an empty asm so the wait for them lands
        // where they are used
        uint32_t rec[kPer];
#pragma unroll
        for (int k = 0; k < kPer; k++) rec[k] = kw[2 * (row - j + min(cl + L * k, j > 0 ? j - 1 : 0u))];
        while (base < n) {
            uint32_t nbase = 0;
            if (lane == 0) nbase = atomicAdd(&next_item, (uint32_t)kSlots);
            nbase = uniform(__shfl(nbase, 0, kWave));
            const uint32_t nmy = nbase + half;
            const bool nhave = nmy < n;
            const uint32_t nrow = nhave ? irow[keys[nmy] & 0xFFFFu] : 0u;
            const uint32_t nj = nhave ? nrow % seq : 0u;
            uint32_t nrec[kPer];
#pragma unroll
            for (int k = 0; k < kPer; k++) nrec[k] = kw[2 * (nrow - nj + min(cl + L * k, nj > 0 ? nj - 1 : 0u))];

            const uint32_t brow = row - j;  // b * S
            // the wavefront walks to its longest item's j; shorter items read the
            // zero row there (adding +0.0 leaves an fp64 sum that starts at +0.0
            // unchanged: it can never be -0.0)
            uint32_t jw = j;
#pragma unroll
            for (int o = L; o < kWave; o <<= 1) jw = max(jw, (uint32_t)__shfl_xor(jw, o, kWave));
            jw = uniform(jw);
            double acc[VW];
#pragma unroll
            for (int c = 0; c < VW; c++) acc[c] = 0.0;
            if constexpr (L == 16) {
                // 16 lanes an item, one DPP row: each lane forms kPer of the chunk's
                // row offsets, and every pair's address add takes its offset from
                // the lane that formed it
                for (uint32_t i0 = 0; i0 < jw; i0 += C) {
                    uint32_t off[kPer];
#pragma unroll
                    for (int k = 0; k < kPer; k++) {
                        const uint32_t i = i0 + cl + L * k;
                        asm volatile("" : "+v"(rec[k]));
                        const uint32_t d = i < j ? j - i - 1 : 0u;
                        off[k] = i < j ? (((((rec[k] & 0xFFFFu) << pe_dim) | ptab[d]) & (sub_rows - 1)) * C) * 4u
                                       : zero_off;
                        rec[k] = kw[2 * (brow + min(i + C, j > 0 ? j - 1 : 0u))];  // next chunk, in flight meanwhile
                    }
                    seq_chunk_add<VW>(tab_b, off, acc, std::make_integer_sequence<int, C / 16>());
                }
            } else
            for (uint32_t i0 = 0; i0 < jw; i0 += C) {
                // this chunk's C row offsets (bytes), kPer per lane
#pragma unroll
                for (int k = 0; k < kPer; k++) {
                    const uint32_t i = i0 + cl + L * k;
                    asm volatile("" : "+v"(rec[k]));
                    const uint32_t d = i < j ? j - i - 1 : 0u;
                    my_rows[cl + L * k] =
                        i < j ? (((((rec[k] & 0xFFFFu) << pe_dim) | ptab[d]) & (sub_rows - 1)) * C) * 4u : zero_off;
                    rec[k] = kw[2 * (brow + min(i + C, j > 0 ? j - 1 : 0u))];  // next chunk, in flight meanwhile
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
                for (int u = 0; u < C; u += 4) {
                    const uint4 r4 = *reinterpret_cast<const uint4 *>(my_rows + u);
                    float v0[VW], v1[VW], v2[VW], v3[VW];
                    lds_cols<VW>(tab_b + r4.x, v0);
                    lds_cols<VW>(tab_b + r4.y, v1);
                    lds_cols<VW>(tab_b + r4.z, v2);
                    lds_cols<VW>(tab_b + r4.w, v3);
#pragma unroll
                    for (int c = 0; c < VW; c++) {
                        acc[c] += (double)v0[c];
                        acc[c] += (double)v1[c];
                        acc[c] += (double)v2[c];
                        acc[c] += (double)v3[c];
                    }
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            }
            if (have && col < n_outputs) {
                uint32_t *dst = part + ((size_t)t * n_rows + row) * n_outputs + col;
#pragma unroll
                for (int c = 0; c < VW; c++) {
                    const uint32_t v = INT_MODE
                        ? (uint32_t)(j > 0 ? (int32_t)(acc[c] * kDenom32 * int_rescaler) : 0)
                        : (j > 0 ? __float_as_uint((float)acc[c]) : 0x80000000u);
                    __builtin_nontemporal_store(v, dst + c);
                }
            }
            base = nbase;
            have = nhave;
            row = nrow;
            j = nj;
#pragma unroll
            for (int k = 0; k < kPer; k++) rec[k] = nrec[k];
        }
    };
    run_chunk(beg, (uint32_t)min((int32_t)kSfItems, end - beg));
    for (int32_t k0 = beg + kSfItems; k0 < end; k0 += kSfItems) {
        const uint32_t n = (uint32_t)min((int32_t)kSfItems, end - k0);
#pragma unroll
        for (int u = 0; u < kSfItems / kSfThreads; u++) {
            const uint32_t it = u * kSfThreads + tid;
            rr[u] = it < n ? (uint32_t)smp[k0 + it] : 0u;
        }
        __syncthreads();  // the previous chunk is done with keys and irow
#pragma unroll
        for (int u = 0; u < kSfItems / kSfThreads; u++) irow[u * kSfThreads + tid] = rr[u];
        run_chunk(k0, n);
    }
}

// ---------------------------------------------------------------------------
// propagate_through_detectors_seq_fc_logic (proto:3629-3835), fp32 summation.
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kRecStage = 512;  // key / positional records an item stages in LDS (j <= 512)

template <int CTRL>
__device__ __forceinline__ void rs16_step(double (&v)[16], int m, bool upper) {
    for (int jj = 0; jj < m; jj++) {
        const double send = upper ? v[jj] : v[m + jj];
        const double keep = upper ? v[m + jj] : v[jj];
        v[jj] = keep + dpp_f64<CTRL>(send);
    }
}

template <int CTRL, int NV>
__device__ __forceinline__ void rs_any(double (&v)[NV], int m, bool upper) {
#pragma unroll
    for (int jj = 0; jj < m; jj++) {
        const double send = upper ? v[jj] : v[m + jj];
        const double keep = upper ? v[m + jj] : v[jj];
        v[jj] = keep + dpp_f64<CTRL>(send);
    }
}

// 16 items per lane, the 8 lanes of a group hold column pieces: afterwards lane
// l holds the group sums of items 2u, 2u+1 with u = 4*(l>=4) + 2*(l&1) + ((l>>1)&1)
// in v[0], v[1].
__device__ __forceinline__ uint32_t rs_pair(uint32_t l) {
    return 4u * (l >= 4 ? 1u : 0u) + 2u * (l & 1u) + ((l >> 1) & 1u);
}

// Two passes, each over (t, b*S + j) items in bucket order, one workgroup per
// item (its wavefronts take the pairs i < j kPB at a time).  Workgroup i runs
// on XCD i % 8 and each XCD takes a contiguous range of items, so the sub-table
// a bucket's items read stays in that XCD's L2 while they run.
//   ALT = false, items bucketed by Q: for each pair, the main row
//     (Q, K_i, P) and, for a K flip, the flipped row (Q, K_i ^ bit, P) and, for
//     a PE flip, (Q, K_i, P ^ bit): fp64 dots with g[b][j] (DPP
//     reduce-scatter), du-scaled and added to dk[b][t][i] / dpe with fp64
//     atomics.  The main rows of the Q-flip pairs are summed instead.
//   ALT = true, items bucketed by Q' = Q ^ (1 << minIdx_j): the flipped rows
//     (Q', K_i, P) of the Q-flip pairs are summed.
// Each pass stores g[b][j] . (its row sum) into qsum[b][t][j]; the Q-flip
// term of (b, t, j) is du(minDelta_j) * (main sum - flipped sum), formed in
// k_seq_xgrad (the reference's per-pair main_grad_sum - alt_grad_sum,
// proto:3740-3783, summed over the pairs first).
// A batch's pair records are decoded by lanes 0..kPB-1 and broadcast with
// readlane; all of its row loads are issued before any of them is used.
constexpr uint32_t kPfMain = 1, kPfK = 2, kPfPe = 4, kPfQ = 8;

template <int NV>
__device__ __forceinline__ void rs_steps(double (&v)[NV], uint32_t l8) {
    // reduce-scatter NV values over the 8 lanes of a group (bits of l8 from
    // the top), then plain sums over the bits left
    if (NV >= 2) rs_any<kDppHalfMirror, NV>(v, NV / 2, l8 >= 4);
    if (NV >= 4) rs_any<kDppXor1, NV>(v, NV / 4, (l8 & 1) != 0);
    if (NV >= 8) rs_any<kDppXor2, NV>(v, NV / 8, ((l8 >> 1) & 1) != 0);
    if (NV < 4) v[0] += dpp_f64<kDppXor1>(v[0]);
    if (NV < 8) v[0] += dpp_f64<kDppXor2>(v[0]);
}

template <int NJ, bool ALT>
__global__ __launch_bounds__(kBlock) void k_propagate_seq(
    const float *__restrict__ w, const float *__restrict__ g, const uint2 *__restrict__ pack,
    const uint2 *__restrict__ ppack, const int32_t *__restrict__ samples, double *__restrict__ qsum,
    double *__restrict__ dk, double *__restrict__ dpe, uint32_t batch, uint32_t seq,
    uint32_t n_outputs, uint32_t n_detectors, uint32_t n_anchors, uint32_t pe_dim,
    uint32_t wg_per_xcd) {
    constexpr int kPB = NJ == 1 ? 4 : (NJ == 2 ? 2 : 1);  // pairs per batch
    constexpr int kNV = 2 * kPB;
    __shared__ double wpart[kWPB];
    __shared__ uint2 srec[kRecStage], sprec[kRecStage];
    const uint32_t lane = threadIdx.x & (kWave - 1);
    const uint32_t wave = uniform(threadIdx.x / kWave);
    const uint32_t n_rows = batch * seq;
    const uint32_t item = (blockIdx.x % 8) * wg_per_xcd + blockIdx.x / 8;
    if (item >= n_detectors * n_rows) return;
    const uint32_t t = item / n_rows;
    const uint32_t row = (uint32_t)samples[item];
    const uint32_t j = row % seq, b = row / seq;
    if (j == 0) return;
    const uint32_t kbits = n_anchors + pe_dim;
    const uint32_t pmask = (1u << pe_dim) - 1;
    const uint2 *kp = pack + (size_t)t * n_rows + (size_t)b * seq;
    const uint2 *pp = ppack + (size_t)t * (seq - 1);
    const float *wt = w + (size_t)t * (1u << (n_anchors + kbits)) * n_outputs;
    const uint2 qr = kp[j];
    const int32_t qm = rec_mi(qr);
    if (ALT && qm < 0) return;
    const uint32_t Q = rec_idx(qr);
    const float qd = rec_md(qr);
    const uint32_t qsub = ALT ? (Q ^ (1u << qm)) : Q;  // the sub-table read
    // the item's key records of positions i < j and positional records of
    // distances d < j, staged once so a batch waits for one L2 trip (its rows)
    const bool staged = j <= (uint32_t)kRecStage;
    if (staged)
        for (uint32_t i = threadIdx.x; i < j; i += kBlock) {
            srec[i] = kp[i];
            sprec[i] = pp[i];
        }
    __syncthreads();

    float gv[NJ][4];
    bool act[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; jj++) {
        const uint32_t c = (jj * kWave + lane) * 4;
        act[jj] = c < n_outputs;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (act[jj]) q = *reinterpret_cast<const float4 *>(g + ((size_t)b * seq + j) * n_outputs + c);
        gv[jj][0] = q.x;
        gv[jj][1] = q.y;
        gv[jj][2] = q.z;
        gv[jj][3] = q.w;
    }
    const uint32_t l8 = lane & 7;
    double rsum[NJ][4];
#pragma unroll
    for (int jj = 0; jj < NJ; jj++)
#pragma unroll
        for (int v = 0; v < 4; v++) rsum[jj][v] = 0.0;

    for (uint32_t i0 = wave * kPB; i0 < j; i0 += kPB * kWPB) {
        const uint32_t n = min((uint32_t)kPB, j - i0);
        // decode the batch's pairs, one per lane
        uint32_t v_main = 0, v_alt = 0, v_pe = 0, v_flags = 0;
        if (lane < n) {
            const uint32_t i = i0 + lane;
            const uint2 kr = staged ? srec[i] : kp[i];
            const uint2 pr = staged ? sprec[j - i - 1] : pp[j - i - 1];
            const uint32_t K = rec_idx(kr), P = rec_idx(pr) & pmask;
            const float kd = rec_md(kr);
            const bool qflip = fabsf(qd) < fabsf(kd);
            v_main = (qsub << kbits) | (K << pe_dim) | P;
            if (ALT) {
                v_flags = qflip ? (kPfMain | kPfQ) : 0u;
            } else {
                const int32_t km = rec_mi(kr), pm = rec_mi(pr);
                const float pdl = rec_md(pr);
                const bool kflip = !qflip && km >= 0;
                const bool peflip = pe_dim > 0 && pm >= 0 && fabsf(pdl) < fabsf(qd) && fabsf(pdl) < fabsf(kd);
                const bool qs = qflip && qm >= 0;
                v_alt = v_main ^ (kflip ? (1u << (km + pe_dim)) : 0u);
                v_pe = v_main ^ (peflip ? (1u << pm) : 0u);
                v_flags = (kflip ? kPfK : 0u) | (peflip ? kPfPe : 0u) | (qs ? kPfQ : 0u);
                if (v_flags) v_flags |= kPfMain;
            }
        }
        f32x4 m[kPB][NJ], a[kPB][NJ], e[kPB][NJ];
        uint32_t fl[kPB];
#pragma unroll
        for (int u = 0; u < kPB; u++) {
            fl[u] = (uint32_t)__builtin_amdgcn_readlane((int)v_flags, u);
            const uint32_t mr = (uint32_t)__builtin_amdgcn_readlane((int)v_main, u);
            const uint32_t ar = (uint32_t)__builtin_amdgcn_readlane((int)v_alt, u);
            const uint32_t er = (uint32_t)__builtin_amdgcn_readlane((int)v_pe, u);
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                const uint32_t c = (jj * kWave + lane) * 4;
                m[u][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
                a[u][jj] = m[u][jj];
                e[u][jj] = m[u][jj];
                if (!act[jj]) continue;
                if (fl[u] & kPfMain) m[u][jj] = *reinterpret_cast<const f32x4 *>(wt + (size_t)mr * n_outputs + c);
                if (!ALT && (fl[u] & kPfK)) a[u][jj] = *reinterpret_cast<const f32x4 *>(wt + (size_t)ar * n_outputs + c);
                if (!ALT && (fl[u] & kPfPe)) e[u][jj] = *reinterpret_cast<const f32x4 *>(wt + (size_t)er * n_outputs + c);
            }
        }
        double items[kNV];
#pragma unroll
        for (int u = 0; u < kPB; u++) {
            double d1 = 0.0, d2 = 0.0;
#pragma unroll
            for (int jj = 0; jj < NJ; jj++) {
                if (fl[u] & kPfQ) {
#pragma unroll
                    for (int v = 0; v < 4; v++) rsum[jj][v] += (double)m[u][jj][v];
                }
                if (!ALT && (fl[u] & kPfK)) {
#pragma unroll
                    for (int v = 0; v < 4; v++) d1 += ((double)m[u][jj][v] - (double)a[u][jj][v]) * (double)gv[jj][v];
                }
                if (!ALT && (fl[u] & kPfPe)) {
#pragma unroll
                    for (int v = 0; v < 4; v++) d2 += ((double)m[u][jj][v] - (double)e[u][jj][v]) * (double)gv[jj][v];
                }
            }
            items[2 * u] = d1;
            items[2 * u + 1] = d2;
        }
        if (ALT) continue;
        rs_steps<kNV>(items, l8);
#pragma unroll
        for (int s = 8; s < kWave; s <<= 1) items[0] += __shfl_xor(items[0], s, kWave);
        // lanes 0..7: value vi of the batch (pair vi / 2; d1 if even, d2 if odd)
        const uint32_t vi = kNV == 8 ? rs_pair(l8) : (kNV == 4 ? 2u * (l8 >= 4 ? 1u : 0u) + (l8 & 1u) : (l8 >= 4 ? 1u : 0u));
        const uint32_t u = vi / 2;
        if (lane < 8 && u < n && (kNV == 8 || (kNV == 4 ? ((l8 >> 1) & 1u) == 0 : (l8 & 3u) == 0))) {
            const uint32_t i = i0 + u;
            const uint2 kr = staged ? srec[i] : kp[i];
            if ((vi & 1u) == 0) {
                const float kd = rec_md(kr);
                if (!(fabsf(qd) < fabsf(kd)) && rec_mi(kr) >= 0)
                    atomicAdd(dk + ((size_t)b * n_detectors + t) * seq + i, du_of_margin(kd) * items[0]);
            } else {
                const uint2 pr = staged ? sprec[j - i - 1] : pp[j - i - 1];
                const int32_t pm = rec_mi(pr);
                const float kd = rec_md(kr), pdl = rec_md(pr);
                if (pe_dim > 0 && pm >= 0 && fabsf(pdl) < fabsf(qd) && fabsf(pdl) < fabsf(kd))
                    atomicAdd(dpe + ((size_t)(j - i - 1) * n_detectors + t) * pe_dim + pm,
                              du_of_margin(pdl) * items[0]);
            }
        }
    }
    // g[b][j] . row sum, over the lanes and then the wavefronts
    double s = 0.0;
#pragma unroll
    for (int jj = 0; jj < NJ; jj++)
#pragma unroll
        for (int v = 0; v < 4; v++) s += rsum[jj][v] * (double)gv[jj][v];
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) s += __shfl_xor(s, o, kWave);
    if (lane == 0) wpart[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = 0.0;
        for (int k = 0; k < kWPB; k++) tot += wpart[k];
        qsum[((size_t)b * n_detectors + t) * seq + j] = tot;
    }
}

// Main pass, pair-parallel form (fp32 summation, O % 4 == 0, O <= kPairMaxO):
// one 256-thread workgroup per (t, b*S + j) item in (t, Q) bucket order
// (XCD-local as above).  g[b][j] is staged in LDS as fp64.  A wavefront takes
// 8 pairs at a time, 8 lanes per pair; lane s of a pair owns the 4-column
// pieces c = 4 * (s + 8k), so each 8-lane group reads 128 contiguous bytes of
// a row per load.  Per pair the lanes form the fp64 dots of g with the main
// row, the K-flipped row (K flips) and the PE-flipped row (PE flips) --
// the reference's main / alt grad sums (proto:3740-3834) over all outputs --
// and reduce them over the 8 lanes with DPP.  Results, without atomics:
//   tk[b][t][j][i] = main - kalt for a K flip, else 0;
//   tp[b][t][j][i] = main - pealt for a PE flip, else 0;
//   qsum[b][t][j]  = sum of main over the Q-flip pairs.
// The triangles are [j*(j-1)/2 + i] per (b, t); k_seq_tri_reduce sums them.
constexpr int kPairMaxO = 2048;  // a multiple of 128 (groups of 4 chunks)
constexpr int kPairChunks = 2;   // 32-column chunks whose rows are loaded together (divides 4)

// fp64 words of g the pair kernel stages: whole groups of 4 chunks of 32 columns
inline uint32_t pair_g_doubles(uint32_t n_outputs) { return ((n_outputs + 31) / 32 + 3) / 4 * 128; }

__global__ __launch_bounds__(kBlock) void k_propagate_seq_pairs(
    const float *__restrict__ w, const float *__restrict__ g, const uint2 *__restrict__ pack,
    const uint2 *__restrict__ ppack, const int32_t *__restrict__ samples, double *__restrict__ qsum,
    double *__restrict__ tk, double *__restrict__ tp, uint32_t batch, uint32_t seq,
    uint32_t n_outputs, uint32_t n_detectors, uint32_t n_anchors, uint32_t pe_dim,
    uint32_t wg_per_xcd) {
    // g in fp64, sized at launch: whole groups of 4 chunks (pair_g_doubles)
    extern __shared__ __attribute__((aligned(16))) double gd[];
    __shared__ double wpart[kWPB];
    __shared__ uint2 srec[kRecStage], sprec[kRecStage];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = uniform(tid / kWave);
    const uint32_t n_rows = batch * seq;
    const uint32_t item = (blockIdx.x % 8) * wg_per_xcd + blockIdx.x / 8;
    if (item >= n_detectors * n_rows) return;
    const uint32_t t = item / n_rows;
    const uint32_t row = (uint32_t)samples[item];
    const uint32_t j = row % seq, b = row / seq;
    if (j == 0) return;
    const uint32_t kbits = n_anchors + pe_dim;
    const uint32_t pmask = (1u << pe_dim) - 1;
    const uint2 *kp = pack + (size_t)t * n_rows + (size_t)b * seq;
    const uint2 *pp = ppack + (size_t)t * (seq - 1);
    const float *wt = w + (size_t)t * (1u << (n_anchors + kbits)) * n_outputs;
    const uint2 qr = kp[j];
    const int32_t qm = rec_mi(qr);
    const uint32_t Q = rec_idx(qr);
    const float qd = rec_md(qr);
    const uint32_t n_chunks = (n_outputs + 31) / 32;  // 32 columns per chunk (8 lanes x 4)
    // g in fp64, zero past the last output up to whole groups of 4 chunks
    // (the clamped loads there add 0)
    for (uint32_t c = tid; c < ((n_chunks + 3) / 4) * 128; c += kBlock)
        gd[c] = c < n_outputs ? (double)g[((size_t)b * seq + j) * n_outputs + c] : 0.0;
    // the item's key and positional records, staged once (one L2 trip per pair
    // batch instead of two)
    const bool staged = j <= (uint32_t)kRecStage;
    if (staged)
        for (uint32_t i = tid; i < j; i += kBlock) {
            srec[i] = kp[i];
            sprec[i] = pp[i];
        }
    __syncthreads();

    const uint32_t p = lane / 8, s = lane % 8;
    const size_t tri = ((size_t)b * n_detectors + t) * ((size_t)seq * (seq - 1) / 2) + (size_t)j * (j - 1) / 2;
    double qacc = 0.0;
    for (uint32_t i0 = wave * 8; i0 < j; i0 += 8 * kWPB) {
        const uint32_t i = i0 + p;
        const bool live = i < j;
        uint32_t mrow = 0, arow = 0, erow = 0;
        bool kflip = false, peflip = false, qs = false;
        if (live) {
            const uint2 kr = staged ? srec[i] : kp[i];
            const uint2 pr = staged ? sprec[j - i - 1] : pp[j - i - 1];
            const uint32_t K = rec_idx(kr), P = rec_idx(pr) & pmask;
            const int32_t km = rec_mi(kr), pm = rec_mi(pr);
            const float kd = rec_md(kr), pdl = rec_md(pr);
            const bool qflip = fabsf(qd) < fabsf(kd);
            kflip = !qflip && km >= 0;
            peflip = pe_dim > 0 && pm >= 0 && fabsf(pdl) < fabsf(qd) && fabsf(pdl) < fabsf(kd);
            qs = qflip && qm >= 0;
            mrow = (Q << kbits) | (K << pe_dim) | P;
            arow = kflip ? (mrow ^ (1u << (km + pe_dim))) : mrow;
            erow = peflip ? (mrow ^ (1u << pm)) : mrow;
        }
        // the flipped rows are loaded only by the pairs that use them (their
        // 8 lanes share the flag, so a skipped row issues no requests); columns
        // past the last output re-read the last 4 and meet g = 0
        double ms = 0.0, as = 0.0, es = 0.0;
        const float *mp = wt + (size_t)mrow * n_outputs;
        const float *ap = wt + (size_t)arow * n_outputs;
        const float *ep = wt + (size_t)erow * n_outputs;
        for (uint32_t k0 = 0; k0 < n_chunks; k0 += kPairChunks) {
            f32x4 mv[kPairChunks], av[kPairChunks], ev[kPairChunks];
#pragma unroll
            for (int k = 0; k < kPairChunks; k++) {
                const uint32_t c = min((k0 + k) * 32 + 4 * s, n_outputs - 4);
                mv[k] = *reinterpret_cast<const f32x4 *>(mp + c);
                av[k] = kflip ? *reinterpret_cast<const f32x4 *>(ap + c) : f32x4{0.f, 0.f, 0.f, 0.f};
                ev[k] = peflip ? *reinterpret_cast<const f32x4 *>(ep + c) : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int k = 0; k < kPairChunks; k++) {
                const uint32_t c = (k0 + k) * 32 + 4 * s;
                const double2 g01 = *reinterpret_cast<const double2 *>(gd + c);
                const double2 g23 = *reinterpret_cast<const double2 *>(gd + c + 2);
                ms += (double)mv[k][0] * g01.x;
                ms += (double)mv[k][1] * g01.y;
                ms += (double)mv[k][2] * g23.x;
                ms += (double)mv[k][3] * g23.y;
                as += (double)av[k][0] * g01.x;
                as += (double)av[k][1] * g01.y;
                as += (double)av[k][2] * g23.x;
                as += (double)av[k][3] * g23.y;
                es += (double)ev[k][0] * g01.x;
                es += (double)ev[k][1] * g01.y;
                es += (double)ev[k][2] * g23.x;
                es += (double)ev[k][3] * g23.y;
            }
        }
        // sums over the 8 lanes of the pair
        ms += dpp_f64<kDppXor1>(ms);
        as += dpp_f64<kDppXor1>(as);
        es += dpp_f64<kDppXor1>(es);
        ms += dpp_f64<kDppXor2>(ms);
        as += dpp_f64<kDppXor2>(as);
        es += dpp_f64<kDppXor2>(es);
        ms += dpp_f64<kDppHalfMirror>(ms);
        as += dpp_f64<kDppHalfMirror>(as);
        es += dpp_f64<kDppHalfMirror>(es);
        if (live && s == 0) {
            tk[tri + i] = kflip ? ms - as : 0.0;
            tp[tri + i] = peflip ? ms - es : 0.0;
            if (qs) qacc += ms;
        }
    }
#pragma unroll
    for (int o = 8; o < kWave; o <<= 1) qacc += __shfl_xor(qacc, o, kWave);
    if (lane == 0) wpart[wave] = qacc;
    __syncthreads();
    if (tid == 0) {
        double tot = 0.0;
        for (int k = 0; k < kWPB; k++) tot += wpart[k];
        qsum[((size_t)b * n_detectors + t) * seq + j] = tot;
    }
}

// One workgroup per (b, t): column sums of tk (the K-flip terms of each
// position i, over the later positions j) and diagonal sums of tp (the PE-flip
// terms of each distance d = j - i - 1).  Position s gets du(minDelta_s) *
// (qsum_main - qsum_alt + column sum); unless |du| <= EPS it goes to
// x_grad[b][s] at the min anchor of (b, s, t) (+du at a1, -du at a2).  The
// diagonal sums times du(pe minDelta) are added to dpe[d][t][pe minIdx].
__global__ __launch_bounds__(kBlock) void k_seq_tri_reduce(
    const double *__restrict__ tk, const double *__restrict__ tp, const double *__restrict__ qs_main,
    const double *__restrict__ qs_alt, const uint2 *__restrict__ pack, const uint2 *__restrict__ ppack,
    const int2 *__restrict__ anchors, float *__restrict__ x_grad, double *__restrict__ dpe,
    uint32_t batch, uint32_t seq, uint32_t n_inputs, uint32_t n_detectors, uint32_t n_anchors,
    uint32_t pe_dim) {
    const uint32_t bt = blockIdx.x;
    const uint32_t b = bt / n_detectors, t = bt % n_detectors;
    const size_t base = (size_t)bt * ((size_t)seq * (seq - 1) / 2);
    for (uint32_t s0 = 0; s0 < seq; s0 += kBlock) {
        const uint32_t s = s0 + threadIdx.x;  // column i = s and diagonal d = s
        double col = 0.0, diag = 0.0;
        if (s < seq) {
#pragma unroll 8
            for (uint32_t jr = s + 1; jr < seq; jr++) {
                const size_t ro = base + (size_t)jr * (jr - 1) / 2;
                col += tk[ro + s];
                diag += tp[ro + (jr - s - 1)];
            }
            const uint2 rec = pack[(size_t)t * batch * seq + (size_t)b * seq + s];
            const size_t q = ((size_t)b * n_detectors + t) * seq + s;
            const double du = du_of_margin(rec_md(rec)) * (qs_main[q] - qs_alt[q] + col);
            const int32_t m = rec_mi(rec);
            if (fabs(du) > kEps && m >= 0 && (uint32_t)m < n_anchors) {
                const int2 a = anchors[(size_t)t * n_anchors + m];
                if ((uint32_t)a.x < n_inputs && (uint32_t)a.y < n_inputs) {
                    float *xg = x_grad + ((size_t)b * seq + s) * n_inputs;
                    unsafeAtomicAdd(xg + a.x, (float)du);
                    unsafeAtomicAdd(xg + a.y, (float)(-du));
                }
            }
            if (pe_dim > 0 && s + 1 < seq && diag != 0.0) {
                const uint2 pr = ppack[(size_t)t * (seq - 1) + s];
                const int32_t pm = rec_mi(pr);
                if (pm >= 0)
                    atomicAdd(dpe + ((size_t)s * n_detectors + t) * pe_dim + pm, du_of_margin(rec_md(pr)) * diag);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Input and positional gradients, LDS-grouped form (fp32 summation, O of 64,
// 128 or 256, Nc <= 10, S <= kGrpMaxDist + 1).
//
// Every (pair i < j, table) term of the reference (proto:3740-3834) is a dot
// of g[b][j] with one to three rows of the (t, Q_j) sub-table: the main row
// (Q_j, K_i, P_d), d = j - i - 1, the K-flipped row (Q_j, K_i ^ bit, P_d) of a
// K flip, the PE-flipped row (Q_j, K_i, P_d ^ bit) of a PE flip; and a Q flip
// dots g[b][j] with the Q-flipped row (Q_j ^ bit, K_i, P_d).  All of those rows
// share their Q with a row of one sub-table, and every flip but the K flip of a
// high bit stays inside a group of 2^gb K values.  So one 1024-thread
// workgroup per (t, Q, K group) stages that group's rows -- 2^(gb + Npe) rows,
// at most 128 KiB -- in LDS once, and computes the dots that read them:
//   main role, the items (b, j) with Q_j = Q (bucket order): for each earlier
//     position i whose K is in the group, the main row (-> qsum of j for a Q
//     flip, -> position i for a K flip, -> distance d for a PE flip), a
//     K-flipped row of a low bit (-> i, negated), a PE-flipped row (-> d,
//     negated); for each earlier i whose K flips to the group by a high bit,
//     the K-flipped row (-> i, negated);
//   Q-flip role, the items with Q_j ^ bit = Q: for each earlier i in the group
//     with a Q flip, the Q-flipped row (-> j, negated).
// Positions come from per-(t, b) lists sorted by group (k_seq_group_lists).
// A wavefront takes one item at a time with g[b][j] in registers (fp32, the
// next item's prefetched into a second set), turns 32 + 16 candidate positions
// a turn (main role; 64 in the Q-flip role) into row dots (a ballot compaction
// into a per-wave LDS queue) and computes 8 dots at a time, 8 lanes a dot: lane
// s of dot slot p reads 16 bytes of each 128-byte chunk, chunks taken in the
// order k ^ (p & 1) so two slots that share a 16-lane LDS cycle read opposite
// bank halves.  Dots are exact fp32 products in fp32 chains and an fp32 tree,
// then fp64; the contributions to j are summed in registers over the item,
// those to i in LDS per candidate (then one fp64 atomic into M[b][t][i] per
// candidate, issued after the next item's loads) and those to d in an LDS sum
// per distance, flushed (times du of the distance's positional margin) into dpe
// once.
// Position s then takes du(minDelta_s) * M[b][t][s] (k_seq_xgrad), the same
// total the pair triangles gave: qsum_main - qsum_alt + the K-flip column sum.

constexpr int kGrpThreads = 1024;
constexpr int kGrpWaves = kGrpThreads / kWave;
constexpr int kGrpTabBytes = 128 * 1024;
constexpr int kGrpMaxDist = 512;   // S - 1
constexpr int kGrpQueue = 128;     // row-dot entries a wave holds (power of two)
constexpr int kGrpMeta = 320;      // items whose metadata a workgroup stages at a time

// Lists of one (t, b): positions of the sequence whose K is in group G
// (list A) and positions whose K flips into group G by a bit >= gb (list B),
// each ascending in i.  Entry: x = the position's minDelta bits,
// y = i | (K & 0x3FF) << 16 | minIdx (0xF: none) << 26.
__global__ __launch_bounds__(kWave) void k_seq_group_lists(
    const uint2 *__restrict__ pack, uint2 *__restrict__ list_a, uint32_t *__restrict__ off_a,
    uint2 *__restrict__ list_b, uint32_t *__restrict__ off_b, uint32_t batch, uint32_t seq,
    uint32_t n_anchors, uint32_t gb) {
    const uint32_t lane = threadIdx.x;
    const uint32_t t = blockIdx.x / batch, b = blockIdx.x % batch;
    const uint32_t ng = 1u << (n_anchors - gb);
    const uint2 *kp = pack + (size_t)t * batch * seq + (size_t)b * seq;
    const size_t lb = (size_t)t * batch + b;
    uint2 *la = list_a + lb * seq, *lbp = list_b + lb * seq;
    uint32_t *oa = off_a + lb * (ng + 1), *ob = off_b + lb * (ng + 1);
    uint32_t na = 0, nb = 0;
    const uint64_t below = (1ull << lane) - 1;
    for (uint32_t G = 0; G < ng; G++) {
        if (lane == 0) {
            oa[G] = na;
            ob[G] = nb;
        }
        for (uint32_t c0 = 0; c0 < seq; c0 += kWave) {
            const uint32_t i = c0 + lane;
            const bool valid = i < seq;
            const uint2 r = valid ? kp[i] : make_uint2(0u, 0u);
            const uint32_t K = rec_idx(r);
            const int32_t km = rec_mi(r);
            const bool in_a = valid && (K >> gb) == G;
            const bool in_b = valid && km >= (int32_t)gb && (uint32_t)km < n_anchors &&
                              ((K ^ (1u << km)) >> gb) == G;
            const uint2 e = make_uint2(r.x, i | ((K & 0x3FFu) << 16) |
                                                ((km < 0 ? 0xFu : (uint32_t)km & 0xFu) << 26));
            const uint64_t ba = __ballot(in_a), bb = __ballot(in_b);
            if (in_a) la[na + __popcll(ba & below)] = e;
            if (in_b) lbp[nb + __popcll(bb & below)] = e;
            na += __popcll(ba);
            nb += __popcll(bb);
        }
    }
    if (lane == 0) {
        oa[ng] = na;
        ob[ng] = nb;
    }
}

// Queue entry (4 bytes): cj | ci << 2 | cd << 4 | (l & 3) << 6 | the row's LDS
// byte offset (bits 8-16: rows of 256 bytes or more in 128 KiB) | d << 17 |
// (l >> 2) << 27, where cj, ci, cd are signed 2-bit coefficients (01 = +1,
// 11 = -1) of the dot's share in position j, position i and distance
// d = j - i - 1, and l is the lane that holds candidate i in its turn.
constexpr uint32_t kCoPlus = 1, kCoMinus = 3;
constexpr int kCoJ = 0, kCoI = 2, kCoD = 4, kEntD = 17;
constexpr uint32_t kEntRow = 0x1FF00u;
__device__ __forceinline__ uint32_t grp_lane_bits(uint32_t l) { return ((l & 3u) << 6) | ((l >> 2) << 27); }
__device__ __forceinline__ uint32_t grp_lane(uint32_t e) { return ((e >> 6) & 3u) | ((e >> 25) & 0x3Cu); }

__device__ __forceinline__ int32_t grp_code(uint32_t e, int at) {
    return __builtin_amdgcn_sbfe((int32_t)e, at, 2);
}

// lanes below this one whose bit is set in a ballot
__device__ __forceinline__ uint32_t lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// v with its sign flipped when bit 0 of s is set
__device__ __forceinline__ double signed_by(double v, uint32_t s) {
    return __longlong_as_double(__double_as_longlong(v) ^ ((long long)(s & 1u) << 63));
}

// a list slot past the end: i = 0xFFFF is >= every j
__device__ __forceinline__ uint2 grp_none() { return make_uint2(0u, 0xFFFFu); }

// fp32 8-lane sum (xor 1, xor 2, half-row mirror), every lane of the group gets it
__device__ __forceinline__ float grp_sum8f(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kDppXor1, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kDppXor2, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kDppHalfMirror, 0xF, 0xF, true));
    return v;
}

// A wavefront's item in the grouped pass: its number in the chunk, its metadata and the
// first candidate of its lists.
struct GrpItem {
    uint32_t it;
    uint4 m;
    uint2 ent;
};

template <int NCH>
__global__ __launch_bounds__(kGrpThreads) void k_propagate_seq_grp(
    const float *__restrict__ w, const float *__restrict__ g, const uint2 *__restrict__ pack,
    const uint2 *__restrict__ ppack, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ samples, const int32_t *__restrict__ offsets2,
    const int32_t *__restrict__ samples2, const uint2 *__restrict__ list_a,
    const uint32_t *__restrict__ off_a, const uint2 *__restrict__ list_b,
    const uint32_t *__restrict__ off_b, double *__restrict__ macc, double *__restrict__ dpe,
    uint32_t batch, uint32_t seq, uint32_t n_detectors, uint32_t n_anchors, uint32_t pe_dim,
    uint32_t gb, uint32_t per_xcd) {
    constexpr uint32_t O = NCH * 32;
    constexpr uint32_t kRowBytes = O * 4;
    __shared__ __attribute__((aligned(16))) uint8_t tab[kGrpTabBytes];
    __shared__ double dsum[kGrpMaxDist];
    __shared__ uint2 prec[kGrpMaxDist];
    __shared__ uint32_t queue[kGrpWaves][kGrpQueue];
    __shared__ uint4 meta[kGrpMeta];
    __shared__ double jtot[kGrpMeta];  // the staged items' own totals
    __shared__ double cacc[kGrpWaves][kWave];  // a turn's position-i sums, one per candidate lane
    __shared__ uint32_t next_item;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = uniform(tid / kWave);
    const uint32_t nq = 1u << n_anchors;
    const uint32_t ng = 1u << (n_anchors - gb);
    const uint32_t wid = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (wid >= n_detectors * nq * ng) return;
    const uint32_t G = wid % ng, Q = (wid / ng) % nq, t = wid / (ng * nq);
    const uint32_t n_rows = batch * seq;
    const int32_t m0 = offsets[(size_t)t * (nq + 1) + Q];
    const int32_t m1 = offsets[(size_t)t * (nq + 1) + Q + 1];
    const int32_t a0 = offsets2[(size_t)t * (2 * nq + 1) + Q];
    const int32_t a1 = offsets2[(size_t)t * (2 * nq + 1) + Q + 1];
    const uint32_t n_main = (uint32_t)(m1 - m0);
    const uint32_t n_items = n_main + (uint32_t)(a1 - a0);
    if (n_items == 0) return;  // uniform over the workgroup
    const uint32_t kbits = n_anchors + pe_dim;
    const uint32_t n_dist = seq - 1;

    // stage the group's rows (one contiguous block of the table)
    {
        const uint32_t bytes = (1u << (gb + pe_dim)) * kRowBytes;
        const uint8_t *src = reinterpret_cast<const uint8_t *>(
            w + ((((size_t)t << n_anchors | Q) << kbits) | ((size_t)G << (gb + pe_dim))) * O);
        for (uint32_t off = wave * kWave * 16; off < bytes; off += kGrpThreads * 16)
            if (off + lane * 16 < bytes)  // groups below 1 KiB: no lane reads past the block
                __builtin_amdgcn_global_load_lds(src + off + lane * 16, (lds_void *)(tab + off), 16, 0, 2);
    }
    for (uint32_t d = tid; d < n_dist; d += kGrpThreads) {
        prec[d] = ppack[(size_t)t * n_dist + d];
        dsum[d] = 0.0;
    }

    const uint32_t p = lane >> 3, s8 = lane & 7;
    const uint32_t podd = p & 1;
    const uint32_t pmask = (1u << pe_dim) - 1, gmask = (1u << gb) - 1;
    uint32_t *q = queue[wave];
    for (uint32_t k = lane; k < kGrpQueue; k += kWave) q[k] = 0;  // a slot past n reads a valid row
    // Position-i shares are summed in LDS per candidate lane (cacc) while a turn
    // runs, then go to M[b][t][i] with one fp64 atomic per lane.  The last turn's
    // sums of an item are flushed at the next item, after its loads are issued:
    // the next wait for loads then finds these atomics long done (the counter it
    // waits on covers atomics too).
    double *const ca = cacc[wave];
    ca[lane] = 0.0;
    size_t fl_base = 0;    // M[b][t][0] of the sums in cacc
    uint32_t fl_i = 0;     // this lane's candidate position of those sums
    bool fl_pend = false;  // cacc holds an item's last turn, not yet flushed
    auto flush = [&]() {
        const double v = ca[lane];
        if (v != 0.0) {
            unsafeAtomicAdd(macc + fl_base + fl_i, v);
            ca[lane] = 0.0;
        }
    };
    // Slot p reads chunk k ^ (p & 1) at turn k, so slots p and p ^ 1 (one
    // 16-lane LDS cycle) read opposite bank halves: even turns from base0 + 128 k,
    // odd turns from base1 + 128 (k - 1) (immediate offsets).  g is held the same way.
    const uint32_t c0l = podd * 128 + 16 * s8;
    const uint32_t c1l = (1 - podd) * 128 + 16 * s8;
    const int32_t *smp = samples + (size_t)t * n_rows + m0;
    const int32_t *smp2 = samples2 + (size_t)t * n_rows + a0;
    const uint2 *kp = pack + (size_t)t * n_rows;

    for (uint32_t c0 = 0; c0 < n_items; c0 += kGrpMeta) {
        const uint32_t cn = min((uint32_t)kGrpMeta, n_items - c0);
        if (c0 > 0) __syncthreads();  // the previous chunk's items are done with meta
        // item metadata: x = row | (qm + 1) << 27, y = qd bits, z = list A range,
        // w = list B range (begin | end << 16, the (t, b) lists of group G)
        for (uint32_t k = tid; k < cn; k += kGrpThreads) {
            const uint32_t it = c0 + k;
            const uint32_t row = (uint32_t)(it < n_main ? smp[it] : smp2[it - n_main]);
            const uint2 qr = kp[row];
            const size_t lb = (size_t)t * batch + row / seq;
            const uint32_t *oa = off_a + lb * (ng + 1);
            const uint32_t *ob = off_b + lb * (ng + 1);
            meta[k] = make_uint4(row | ((uint32_t)(rec_mi(qr) + 1) << 27), qr.x, oa[G] | (oa[G + 1] << 16),
                                 ob[G] | (ob[G + 1] << 16));
            jtot[k] = 0.0;
        }
        if (tid == 0) next_item = 0;
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the table block too
        __syncthreads();

        auto fetch = [&]() -> uint32_t {
            uint32_t v = 0;
            if (lane == 0) v = atomicAdd(&next_item, 1u);
            return uniform(v);  // lane 0 is the first active lane here
        };
        // an item's loads: g[b][j] in this lane's chunk order and the first
        // candidate of its lists (main role: lanes 0-31 list A, 32-47 list B;
        // Q-flip role: every lane list A)
        auto issue = [&](uint32_t k, uint4 &mm, float (&gg)[NCH][4]) -> uint2 {
            mm = meta[k];
            const uint32_t row = mm.x & 0x7FFFFFFu;
            const bool main_r = c0 + k < n_main;
            const float *g0 = g + (size_t)row * O + c0l / 4;
            const float *g1 = g + (size_t)row * O + c1l / 4;
#pragma unroll
            for (int kk = 0; kk < NCH; kk++) {
                const f32x4 v = (kk & 1) ? *reinterpret_cast<const f32x4 *>(g1 + (kk - 1) * 32)
                                         : *reinterpret_cast<const f32x4 *>(g0 + kk * 32);
#pragma unroll
                for (int c = 0; c < 4; c++) gg[kk][c] = v[c];
            }
            const bool use_b = main_r && lane >= 32;
            const uint32_t rng = use_b ? mm.w : mm.z;
            const uint32_t cur = (rng & 0xFFFFu) + (use_b ? lane - 32 : lane);
            const bool in = (!main_r || lane < 48) && cur < (rng >> 16);
            const size_t lb = (size_t)t * batch + row / seq;
            return in ? (use_b ? list_b : list_a)[lb * seq + cur] : grp_none();
        };

        // One visit: item cur with its g in gf; the next item's loads go to gn.  The
        // loop alternates the two register sets, so no copy moves g between them.
        auto visit = [&](const GrpItem cur, float (&gf)[NCH][4], float (&gn)[NCH][4]) -> GrpItem {
            const uint32_t it = cur.it;
            const uint4 m = cur.m;
            // wait for this item's loads before the next item's are issued: the
            // counter then covers them alone
#pragma unroll
            for (int k = 0; k < NCH; k++)
#pragma unroll
                for (int c = 0; c < 4; c++) __asm__ volatile("" : "+v"(gf[k][c]));
            uint32_t ex = cur.ent.x, ey = cur.ent.y;
            __asm__ volatile("" : "+v"(ex), "+v"(ey));
            const uint2 ent = make_uint2(ex, ey);
            GrpItem nx;
            nx.it = fetch();
            nx.m = make_uint4(0u, 0u, 0u, 0u);
            nx.ent = grp_none();
            if (nx.it < cn) nx.ent = issue(nx.it, nx.m, gn);
            if (fl_pend) {  // the previous item's last turn
                flush();
                fl_pend = false;
            }

            const bool main_role = c0 + it < n_main;
            const uint32_t row = m.x & 0x7FFFFFFu;
            const uint32_t b = row / seq, j = row % seq;
            const int32_t qm = (int32_t)(m.x >> 27) - 1;
            const float qd = __uint_as_float(m.y);
            if (j > 0) {
                const size_t mbase = ((size_t)b * n_detectors + t) * seq;
                double jacc = 0.0;
                uint32_t qh = 0, qt = 0;

                // 8 row dots from the queue (n of them live): exact fp32 products
                // (FMA) in four fp32 chains of NCH terms per lane, the chains and
                // the slot's 8 lanes summed in fp32 (a tree of depth 5), the dot
                // then in fp64.  Slots past n read a stale entry's row (the ring
                // starts zeroed) and add nothing.
                auto step = [&](uint32_t n, auto main_tag) {
                    constexpr bool kMain = decltype(main_tag)::value;
                    const uint32_t e = q[(qh + p) & (kGrpQueue - 1)];
                    const bool on = p < n;
                    const uint8_t *t0 = tab + ((e & kEntRow) | c0l);
                    const uint8_t *t1 = tab + ((e & kEntRow) | c1l);
                    float f0 = 0.f, f1 = 0.f, f2 = 0.f, f3 = 0.f;
#pragma unroll
                    for (int k = 0; k < NCH; k++) {
                        const f32x4 v = (k & 1) ? *reinterpret_cast<const f32x4 *>(t1 + (k - 1) * 128)
                                                : *reinterpret_cast<const f32x4 *>(t0 + k * 128);
                        f0 = fmaf(v[0], gf[k][0], f0);
                        f1 = fmaf(v[1], gf[k][1], f1);
                        f2 = fmaf(v[2], gf[k][2], f2);
                        f3 = fmaf(v[3], gf[k][3], f3);
                    }
                    const float part = on ? (f0 + f1) + (f2 + f3) : 0.f;
                    const double tot = (double)grp_sum8f(part);
                    if constexpr (!kMain) {
                        jacc -= tot;  // Q-flip entries: cj = -1, no other share
                    } else {
                        jacc += (double)grp_code(e, kCoJ) * tot;  // the same in the group's 8 lanes
                        const bool pushes = on && (e & (0xFu << kCoI)) != 0;
                        if (__builtin_amdgcn_ballot_w64(pushes)) {
                            if (pushes && s8 == 0) {
                                const int32_t ci = grp_code(e, kCoI), cd = grp_code(e, kCoD);
                                // a share is +-tot: the code's high bit is the sign
                                if (ci) atomicAdd(&ca[grp_lane(e)], signed_by(tot, e >> (kCoI + 1)));
                                if (cd) atomicAdd(&dsum[(e >> kEntD) & 0x3FFu], signed_by(tot, e >> (kCoD + 1)));
                            }
                        }
                    }
                    qh += n;
                };

                const size_t lb = (size_t)t * batch + b;
                auto run_lists = [&](auto main_tag) {
                    constexpr bool kMain = decltype(main_tag)::value;
                    const bool use_b = kMain && lane >= 32;
                    const bool lane_on = !kMain || lane < 48;
                    const uint32_t span = kMain ? (use_b ? 16u : 32u) : 64u;
                    const uint32_t rng = use_b ? m.w : m.z;
                    uint32_t cur = (rng & 0xFFFFu) + (use_b ? lane - 32 : lane);
                    const uint32_t end = rng >> 16;
                    const uint2 *lst = (use_b ? list_b : list_a) + lb * seq;
                    uint2 r = ent;  // the first candidate, loaded with the item
                    for (;;) {
                        const uint32_t i = r.y & 0xFFFFu;
                        const bool valid = i < j;  // slots past a list's end carry i = 0xFFFF
                        if (__ballot(valid) == 0) break;  // ascending i: the rest are >= j
                        uint32_t n_rd = 0, e_a = 0, e_b = 0, e_c = 0;
                        if (valid) {
                            const uint32_t K = (r.y >> 16) & 0x3FFu;
                            const float kd = __uint_as_float(r.x);
                            const uint2 pr = prec[j - i - 1];
                            const uint32_t P = rec_idx(pr) & pmask;
                            const bool qflip = fabsf(qd) < fabsf(kd);
                            const uint32_t iw = ((j - i - 1) << kEntD) | grp_lane_bits(lane);
                            const uint32_t lrow = (((K & gmask) << pe_dim) | P) * kRowBytes;
                            if constexpr (!kMain) {  // Q-flip role (qm >= 0 for these items)
                                e_a = lrow | (kCoMinus << kCoJ) | iw;
                                n_rd = qflip ? 1u : 0u;
                            } else {
                                const uint32_t kmc = r.y >> 26;
                                const int32_t km = kmc == 0xFu ? -1 : (int32_t)kmc;
                                if (use_b) {  // a K flip of a bit >= gb into this group
                                    e_a = (((((K ^ (1u << (km & 31))) & gmask) << pe_dim) | P) * kRowBytes) | (kCoMinus << kCoI) | iw;
                                    n_rd = qflip ? 0u : 1u;
                                } else {
                                    const int32_t pm = rec_mi(pr);
                                    const float pdl = rec_md(pr);
                                    const bool kflip = !qflip && km >= 0;
                                    const bool peflip = pe_dim > 0 && pm >= 0 && fabsf(pdl) < fabsf(qd) &&
                                                        fabsf(pdl) < fabsf(kd);
                                    const bool qs = qflip && qm >= 0;
                                    const bool low_k = kflip && (uint32_t)km < gb;
                                    e_a = lrow | ((qs ? kCoPlus : 0u) << kCoJ) | ((kflip ? kCoPlus : 0u) << kCoI) |
                                          ((peflip ? kCoPlus : 0u) << kCoD) | iw;
                                    const uint32_t e_k = (lrow ^ (kRowBytes << ((km + pe_dim) & 31))) | (kCoMinus << kCoI) | iw;
                                    const uint32_t e_p = (lrow ^ (kRowBytes << (pm & 31))) | (kCoMinus << kCoD) | iw;
                                    e_b = low_k ? e_k : e_p;
                                    e_c = e_p;
                                    n_rd = (qs || kflip || peflip) ? 1u + (low_k ? 1u : 0u) + (peflip ? 1u : 0u) : 0u;
                                }
                            }
                        }
                        const uint64_t b1 = __ballot(n_rd >= 1);
                        const uint64_t b2 = kMain ? __ballot(n_rd >= 2) : 0ull;
                        const uint64_t b3 = kMain ? __ballot(n_rd >= 3) : 0ull;
                        const uint32_t pos = qt + lanes_below(b1) + (kMain ? lanes_below(b2) + lanes_below(b3) : 0u);
                        if (n_rd >= 1) q[pos & (kGrpQueue - 1)] = e_a;
                        if (kMain && n_rd >= 2) q[(pos + 1) & (kGrpQueue - 1)] = e_b;
                        if (kMain && n_rd >= 3) q[(pos + 2) & (kGrpQueue - 1)] = e_c;
                        qt += __popcll(b1) + __popcll(b2) + __popcll(b3);
                        cur += span;
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        while (qt - qh >= 8) step(8, main_tag);
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        if constexpr (kMain) {
                            fl_i = i;  // cacc[lane] sums this turn's candidate
                            if (__builtin_amdgcn_ballot_w64(lane_on && cur < end)) {
                                // another turn follows: finish this one and flush its sums
                                while (qt != qh) step(min(8u, qt - qh), main_tag);
                                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                                __builtin_amdgcn_wave_barrier();
                                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                                fl_base = mbase;
                                flush();
                            }
                        }
                        // lists longer than a turn: wait for the reload here, so the loop
                        // head holds no wait that would cover the next item's loads
                        r = (lane_on && cur < end) ? lst[cur] : grp_none();
                        uint32_t rx = r.x, ry = r.y;
                        __asm__ volatile("" : "+v"(rx), "+v"(ry));
                        r = make_uint2(rx, ry);
                    }
                    if (qt != qh) step(qt - qh, main_tag);
                    if constexpr (kMain) {
                        fl_base = mbase;
                        fl_pend = true;
                    }
                };
                if (main_role)
                    run_lists(std::integral_constant<bool, true>());
                else
                    run_lists(std::integral_constant<bool, false>());
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                // the item's own total: one value per slot group (its 8 lanes agree), summed
                // over the groups by a row rotation and four lane reads (no LDS round trip)
                const double pair = jacc + dpp_f64<0x128>(jacc);  // row_ror:8, the row's other group
                const double jsum = (readlane_f64(pair, 0) + readlane_f64(pair, 16)) +
                                    (readlane_f64(pair, 32) + readlane_f64(pair, 48));
                if (lane == 0) jtot[it] = jsum;  // flushed with the chunk: no atomic before the next item's wait
            }
            return nx;
        };

        float gr0[NCH][4], gr1[NCH][4];
        GrpItem cur;
        cur.it = fetch();
        cur.m = make_uint4(0u, 0u, 0u, 0u);
        cur.ent = grp_none();
        if (cur.it < cn) cur.ent = issue(cur.it, cur.m, gr0);
        while (cur.it < cn) {
            cur = visit(cur, gr0, gr1);
            if (cur.it >= cn) break;
            cur = visit(cur, gr1, gr0);
        }
        if (fl_pend) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            flush();
            fl_pend = false;
        }
        __syncthreads();
        // the chunk's item totals
        for (uint32_t k = tid; k < cn; k += kGrpThreads) {
            const double v = jtot[k];
            if (v != 0.0) {
                const uint32_t row = meta[k].x & 0x7FFFFFFu;
                unsafeAtomicAdd(macc + ((size_t)(row / seq) * n_detectors + t) * seq + row % seq, v);
            }
        }
    }
    __syncthreads();
    // distance sums, scaled by du of the distance's positional margin
    for (uint32_t d = tid; d < n_dist; d += kGrpThreads) {
        const double v = dsum[d];
        if (v != 0.0) {
            const uint2 pr = prec[d];
            const int32_t pm = rec_mi(pr);
            if (pm >= 0)
                unsafeAtomicAdd(dpe + ((size_t)d * n_detectors + t) * pe_dim + pm, du_of_margin(rec_md(pr)) * v);
        }
    }
}

// Exact decomposition: one thread per (b, t, pair, output block).
template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_propagate_seq_exact(
    const float *__restrict__ w, const float *__restrict__ g, const uint2 *__restrict__ pack,
    const uint2 *__restrict__ ppack, const int2 *__restrict__ anchors, float *__restrict__ x_grad,
    float *__restrict__ pe_grad, uint32_t batch, uint32_t seq, uint32_t n_inputs,
    uint32_t n_outputs, uint32_t n_detectors, uint32_t n_anchors, uint32_t pe_dim, uint32_t ogs,
    uint32_t n_ob, uint64_t n_items, double int_rescaler) {
    const uint64_t item = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (item >= n_items) return;
    const uint64_t n_pairs = (uint64_t)seq * (seq - 1) / 2;
    const uint32_t ob = (uint32_t)(item % n_ob);
    const uint64_t r1 = item / n_ob;
    const uint64_t p = r1 % n_pairs;
    const uint64_t r2 = r1 / n_pairs;
    const uint32_t t = (uint32_t)(r2 % n_detectors);
    const uint32_t b = (uint32_t)(r2 / n_detectors);
    // pair p -> (i < j): j is the largest with j*(j-1)/2 <= p
    uint32_t j = (uint32_t)((1.0 + sqrt(1.0 + 8.0 * (double)p)) * 0.5);
    while ((uint64_t)j * (j - 1) / 2 > p) j--;
    while ((uint64_t)(j + 1) * j / 2 <= p) j++;
    const uint32_t i = (uint32_t)(p - (uint64_t)j * (j - 1) / 2);
    const uint32_t n_rows = batch * seq;
    const uint32_t kbits = n_anchors + pe_dim;
    const uint32_t pmask = (1u << pe_dim) - 1;
    const uint2 *kp = pack + (size_t)t * n_rows + (size_t)b * seq;
    const uint2 qr = kp[j], kr = kp[i];
    const uint2 pr = ppack[(size_t)t * (seq - 1) + (j - i - 1)];
    const uint32_t Q = rec_idx(qr), K = rec_idx(kr), P = rec_idx(pr) & pmask;
    const int32_t qm = rec_mi(qr), km = rec_mi(kr), pm = rec_mi(pr);
    const float qd = rec_md(qr), kd = rec_md(kr), pdl = rec_md(pr);
    const bool qflip = fabsf(qd) < fabsf(kd);
    const int32_t fm = qflip ? qm : km;
    const uint32_t main_row = (Q << kbits) | (K << pe_dim) | P;
    const uint32_t alt_row = fm < 0 ? main_row
                                    : (qflip ? (main_row ^ (1u << (fm + kbits)))
                                             : (main_row ^ (1u << (fm + pe_dim))));
    const float *wt = w + (size_t)t * (1u << (n_anchors + kbits)) * n_outputs;
    const float *gj = g + ((size_t)b * seq + j) * n_outputs;
    const uint32_t o0 = ob * ogs, o1 = min(o0 + ogs, n_outputs);
    double ms = 0.0, as = 0.0;
    for (uint32_t o = o0; o < o1; o++) {
        const double gg = (double)gj[o];
        ms += (double)wt[(size_t)main_row * n_outputs + o] * gg;
        as += (double)wt[(size_t)alt_row * n_outputs + o] * gg;
    }
    if (fm >= 0) {
        const double du = du_of_margin(qflip ? qd : kd) * (ms - as);
        if (fabs(du) > kEps) {
            const int2 a = anchors[(size_t)t * n_anchors + fm];
            if ((uint32_t)a.x < n_inputs && (uint32_t)a.y < n_inputs) {
                float *xg = x_grad + ((size_t)b * seq + (qflip ? j : i)) * n_inputs;
                if (INT_MODE) {
                    const int32_t d = (int32_t)(du * kDenom32 * int_rescaler);
                    atomicAdd(reinterpret_cast<int32_t *>(xg + a.x), d);
                    atomicAdd(reinterpret_cast<int32_t *>(xg + a.y), (int32_t)(0u - (uint32_t)d));
                } else {
                    unsafeAtomicAdd(xg + a.x, (float)du);
                    unsafeAtomicAdd(xg + a.y, (float)(-du));
                }
            }
        }
    }
    if (pe_dim > 0 && pm >= 0 && fabsf(pdl) < fabsf(qd) && fabsf(pdl) < fabsf(kd)) {
        const uint32_t pe_row = main_row ^ (1u << pm);
        double es = 0.0;
        for (uint32_t o = o0; o < o1; o++)
            es += (double)wt[(size_t)pe_row * n_outputs + o] * (double)gj[o];
        const double dpe = du_of_margin(pdl) * (ms - es);
        float *dst = pe_grad + ((size_t)(j - i - 1) * n_detectors + t) * pe_dim + pm;
        if (INT_MODE)
            atomicAdd(reinterpret_cast<int32_t *>(dst), (int32_t)(dpe * kDenom32 * int_rescaler));
        else
            unsafeAtomicAdd(dst, (float)dpe);
    }
}

// Bucket key of the Q-flip pass: Q ^ (1 << minIdx), or 2^Nc (a bin past every
// sub-table) when no anchor can flip.
__global__ __launch_bounds__(kBlock) void k_seq_alt_keys(const int32_t *__restrict__ idx,
                                                         const int32_t *__restrict__ mi,
                                                         int32_t *__restrict__ keys, uint64_t n,
                                                         uint32_t n_anchors) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i >= n) return;
    const int32_t m = mi[i];
    keys[i] = (m >= 0 && (uint32_t)m < n_anchors) ? (int32_t)(((uint32_t)idx[i] ^ (1u << m)) & ((1u << n_anchors) - 1))
                                                   : (int32_t)(1u << n_anchors);
}

// x_grad[b][s][a1] += du, [a2] -= du with du = du(minDelta) * (qsum_main -
// qsum_alt) + dk of (b, t, s) and the min anchor of (b, s, t) (both the Q flips
// at s and the K flips at s flip that anchor), dropped unless |du| > EPS.
// qsum_alt and dk may be null (the grouped pass leaves one total in qsum_main).
__global__ __launch_bounds__(kBlock) void k_seq_xgrad(const double *__restrict__ qs_main,
                                                      const double *__restrict__ qs_alt,
                                                      const double *__restrict__ dk,
                                                      const uint2 *__restrict__ pack,
                                                      const int2 *__restrict__ anchors,
                                                      float *__restrict__ x_grad, uint32_t batch,
                                                      uint32_t seq, uint32_t n_inputs,
                                                      uint32_t n_detectors, uint32_t n_anchors) {
    const uint64_t it = (uint64_t)blockIdx.x * kBlock + threadIdx.x;  // (b, t, s)
    const uint64_t n = (uint64_t)batch * n_detectors * seq;
    if (it >= n) return;
    const uint32_t s = (uint32_t)(it % seq);
    const uint32_t t = (uint32_t)((it / seq) % n_detectors);
    const uint32_t b = (uint32_t)(it / ((uint64_t)seq * n_detectors));
    const uint2 rec = pack[(size_t)t * batch * seq + (size_t)b * seq + s];
    const double du = du_of_margin(rec_md(rec)) * (qs_main[it] - (qs_alt ? qs_alt[it] : 0.0)) +
                      (dk ? dk[it] : 0.0);
    if (!(fabs(du) > kEps)) return;
    const int32_t m = rec_mi(rec);
    if (m < 0 || (uint32_t)m >= n_anchors) return;
    const int2 a = anchors[(size_t)t * n_anchors + m];
    if ((uint32_t)a.x >= n_inputs || (uint32_t)a.y >= n_inputs) return;
    float *xg = x_grad + ((size_t)b * seq + s) * n_inputs;
    unsafeAtomicAdd(xg + a.x, (float)du);
    unsafeAtomicAdd(xg + a.y, (float)(-du));
}

// pe_grad (+)= fp32(accumulated fp64 terms).
__global__ __launch_bounds__(kBlock) void k_seq_pe_commit(const double *__restrict__ dpe,
                                                          float *__restrict__ pe_grad, uint32_t n) {
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) pe_grad[i] = (float)((double)pe_grad[i] + dpe[i]);
}

__global__ __launch_bounds__(kBlock) void k_zero64(double *__restrict__ p, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (i < n) p[i] = 0.0;
}

// ---------------------------------------------------------------------------
// gather_w_gradients_seq_fc (proto:3944-4304), one workgroup per (table t,
// Q value q).  The items (b, j) of the bucket (t, q) are taken in batches; a
// batch's (item, earlier position i) entries are bucketed by their target row
// (K_i, PE_{j-i-1}) once (LDS counting sort), then for each column slice of C
// columns the batch's gradient rows are staged in LDS and every thread sums
// the commit values of its 32 (row, column) outputs' entries in registers and
// writes them (the first batch stores or adds as asked, later ones add).  No
// floating-point atomics and, for a bucket of one batch, each weight-gradient
// element is written once (the zero-fill of the caller's buffer is fused
// away).  fp32 sums come in bucket order rather than the reference CPU path's
// order; int32 payload sums are exact.
constexpr int kSeqWgThreads = 1024;
constexpr int kSeqWgRowsMax = 4096;      // sub-table rows 2^(Nc+Npe)
// LDS: 32 KiB of row counts and cursors, 52 KiB of u8 entries, 49 KiB of
// gradient rows, 19 KiB of index tables: 195 items of 255 earlier positions (and
// the pads of 1024 rows)
// and 64 columns fit one batch, so a (table, Q) bucket of up to 195 items --
// every bucket of 2^6 Q values over 8192 (b, s) rows in practice -- is summed
// and written in one pass.  A row's bucket of entries is padded to a multiple
// of four (pads name the zero row), so the walk reads entries four at a time.
constexpr int kSeqWgEntries = 53248;     // entries per batch (u8 item numbers), pads included
constexpr int kSeqWgGvWords = 12544;     // batch gradient rows (items x C) and the zero row
constexpr int kSeqWgKeys = 8192;         // K indices of up to 8192 (b, s) rows at a time
constexpr int kSeqWgPe = 1024;
constexpr int kSeqWgItems = 256;         // u8 entries: at most 256 items a batch
constexpr int kQuadStep = 4;             // entries a turn of the 16-byte row loop (one u32 read)
constexpr int kSeqWgClasses = 64;        // row length classes (turns of kQuadStep entries, the last open)
// The wide walk (128 columns a pass, two 64-column planes of gradient rows) fits
// LDS for sub-tables of up to 1024 rows: its second plane shares its array with
// the K and positional index tables, which a batch's walk does not read.
constexpr int kSeqWgWideRows = 1024;
static_assert(kSeqWgGvWords * 4 >= (kSeqWgKeys + kSeqWgPe) * 2, "the index tables fit the second plane");

// The order in which the weight gradient's workgroups take the (table, Q)
// buckets: largest first (classes of 32 items), so that the longest workgroups
// -- buckets past one batch, where an input's few values concentrate its Q --
// start first instead of trailing the grid.  One workgroup.
constexpr int kOrderClasses = 64;
constexpr uint32_t kOrderMaxBuckets = 65536;  // beyond: table order (one workgroup sorts)
__global__ __launch_bounds__(kSeqWgThreads) void k_bucket_order(const int32_t *__restrict__ offsets,
                                                              uint32_t n_q, uint32_t n_buckets,
                                                              uint32_t *__restrict__ order) {
    __shared__ uint32_t hist[kOrderClasses];
    const uint32_t tid = threadIdx.x;
    auto cls = [&](uint32_t b) -> uint32_t {
        const int32_t *o = offsets + (size_t)(b / n_q) * (n_q + 1) + b % n_q;
        const uint32_t n = (uint32_t)(o[1] - o[0]);
        return (uint32_t)kOrderClasses - 1u - min(n / 32u, (uint32_t)kOrderClasses - 1u);
    };
    if (tid < (uint32_t)kOrderClasses) hist[tid] = 0u;
    __syncthreads();
    for (uint32_t b = tid; b < n_buckets; b += kSeqWgThreads) atomicAdd(&hist[cls(b)], 1u);
    __syncthreads();
    if (tid < (uint32_t)kWave) {  // exclusive scan of the class counts
        const uint32_t v = tid < (uint32_t)kOrderClasses ? hist[tid] : 0u;
        uint32_t incl = v;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const uint32_t y = __shfl_up(incl, o, kWave);
            if ((int)tid >= o) incl += y;
        }
        if (tid < (uint32_t)kOrderClasses) hist[tid] = incl - v;
    }
    __syncthreads();
    for (uint32_t b = tid; b < n_buckets; b += kSeqWgThreads) order[atomicAdd(&hist[cls(b)], 1u)] = b;
}

template <bool INT_MODE, bool OVERWRITE, bool WIDE>
__global__ __launch_bounds__(kSeqWgThreads) void k_wgrad_seq_sort(
    const uint32_t *__restrict__ cv, const int32_t *__restrict__ offsets,
    const int32_t *__restrict__ samples, const uint2 *__restrict__ pack,
    const uint2 *__restrict__ ppack, const uint32_t *__restrict__ order, float *__restrict__ target,
    uint32_t batch, uint32_t seq, uint32_t n_outputs, uint32_t n_detectors, uint32_t n_anchors,
    uint32_t pe_dim, uint32_t cols, uint32_t n_slices, uint32_t items_per_batch, double int_rescaler,
    bool quad) {
    constexpr int kRowsCap = WIDE ? kSeqWgWideRows : kSeqWgRowsMax;
    __shared__ uint32_t cnt[kRowsCap + 1];  // counts, then (quad path) the walk's words and its end
    __shared__ uint32_t cur[kRowsCap];
    __shared__ __attribute__((aligned(4))) uint8_t ent[kSeqWgEntries + 2 * kQuadStep];  // + the walk's read-ahead
    __shared__ __attribute__((aligned(16))) uint32_t gv[kSeqWgGvWords];
    // the wide walk's second column plane, which also holds the index tables
    // while a batch is sorted
    __shared__ __attribute__((aligned(16))) uint32_t gv_hi[WIDE ? kSeqWgGvWords : 1];
    __shared__ uint16_t ktab_own[WIDE ? 1 : kSeqWgKeys];
    __shared__ uint16_t ptab_own[WIDE ? 1 : kSeqWgPe];
    uint16_t *const ktab = WIDE ? reinterpret_cast<uint16_t *>(gv_hi) : ktab_own;
    uint16_t *const ptab = WIDE ? reinterpret_cast<uint16_t *>(gv_hi) + kSeqWgKeys : ptab_own;
    __shared__ uint32_t bitems[kSeqWgItems];  // row ids of the batch's items
    __shared__ uint32_t wsum[kSeqWgThreads / kWave];
    __shared__ uint32_t lhist[kSeqWgClasses];  // rows per length class (quad path)
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = tid / kWave;
    const uint32_t n_q = 1u << n_anchors;
    const uint32_t bq = order ? order[blockIdx.x] : blockIdx.x;  // the bucket (t, q), largest first
    const uint32_t t = bq / n_q, q = bq % n_q;
    const uint32_t sub_rows = 1u << (n_anchors + pe_dim);
    const uint32_t pmask = (1u << pe_dim) - 1;
    const uint32_t n_rows = batch * seq;
    const uint32_t my_col = tid % cols;  // cols divides the 1024 threads

    auto load_ptab = [&]() {
        for (uint32_t d = tid; d + 1 < seq; d += kSeqWgThreads)
            ptab[d] = (uint16_t)(rec_idx(ppack[(size_t)t * (seq - 1) + d]) & pmask);
    };
    if (!WIDE) load_ptab();
    const int32_t *off_t = offsets + (size_t)t * (n_q + 1);
    const int32_t beg = off_t[q], end = off_t[q + 1];
    const int32_t *smp = samples + (size_t)t * n_rows;
    const uint2 *kp = pack + (size_t)t * n_rows;
    const uint32_t rows_per_chunk = (kSeqWgKeys / seq) * seq;
    float *dst = target + ((size_t)t * n_q + q) * sub_rows * n_outputs;

    bool first = true;
    int32_t k0 = beg;
    for (uint32_t r0 = 0; r0 < n_rows && k0 < end; r0 += rows_per_chunk) {
        const uint32_t r1 = min(r0 + rows_per_chunk, n_rows);
        __syncthreads();
        // the chunk's K indices, eight loads in flight a thread
        auto load_ktab = [&]() {
            for (uint32_t r = r0 + tid; r < r1; r += 8 * kSeqWgThreads) {
                uint32_t kv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t rr = r + u * kSeqWgThreads;
                    kv[u] = rr < r1 ? kp[rr].y : 0u;
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t rr = r + u * kSeqWgThreads;
                    if (rr < r1) ktab[rr - r0] = (uint16_t)rec_idx(make_uint2(0u, kv[u]));
                }
            }
        };
        if (!WIDE) load_ktab();
        // first bucket position at or past row r1 (uniform binary search; the
        // bucket's end when the chunk reaches the last row)
        int32_t lo = k0, hi = end;
        if (r1 >= n_rows) lo = end;
        while (lo < hi) {
            const int32_t mid = lo + (hi - lo) / 2;
            if ((uint32_t)smp[mid] < r1) lo = mid + 1; else hi = mid;
        }
        const int32_t k1 = lo;
        for (int32_t kb = k0; kb < k1; kb += (int32_t)items_per_batch) {
            const uint32_t nb = (uint32_t)min((int32_t)items_per_batch, k1 - kb);
            __syncthreads();
            // the batch's items; zero counts; (wide walk) the index tables, which
            // the previous batch's walk overwrote
            if (WIDE) {
                load_ptab();
                load_ktab();
            }
            for (uint32_t it = tid; it < nb; it += kSeqWgThreads) bitems[it] = (uint32_t)smp[kb + it];
            for (uint32_t r = tid; r < sub_rows; r += kSeqWgThreads) cnt[r] = 0u;
            __syncthreads();
            // count: one wavefront per item, lanes over earlier positions i
            for (uint32_t it = wave; it < nb; it += kSeqWgThreads / kWave) {
                const uint32_t r = bitems[it];
                const uint32_t j = r % seq;
                const uint16_t *kt = ktab + (r / seq - r0 / seq) * seq;
                for (uint32_t i = lane; i < j; i += kWave)
                    atomicAdd(&cnt[(((uint32_t)kt[i] << pe_dim) | ptab[j - i - 1]) & (sub_rows - 1)], 1u);
            }
            __syncthreads();
            // Bucket starts, padded to whole turns of kQuadStep entries.  The quad
            // path lays the buckets out in its walk order (rows by length class,
            // longest first, so the four 16-lane groups of a wavefront reach
            // their rows' ends on the same turn): a walk position's bucket then
            // runs from its start to the next position's, and the walk reads one
            // packed word a position, cnt[pos] = row | start / 4 << 12 (written
            // over the counts once they are read; cnt[sub_rows] = the end).  The
            // other path keeps row order.  cur[row] = the row's start, the
            // scatter's cursor.
            constexpr int kRowPasses = kSeqWgRowsMax / kSeqWgThreads;
            auto row_class = [&](uint32_t r) -> uint32_t {
                const uint32_t turns = (cnt[r] + kQuadStep - 1) / kQuadStep;
                return (uint32_t)kSeqWgClasses - 1u - min(turns, (uint32_t)kSeqWgClasses - 1u);
            };
            if (quad) {
                for (uint32_t c = tid; c < (uint32_t)kSeqWgClasses; c += kSeqWgThreads) lhist[c] = 0u;
                __syncthreads();
                for (uint32_t r = tid; r < sub_rows; r += kSeqWgThreads) atomicAdd(&lhist[row_class(r)], 1u);
                __syncthreads();
                if (wave == 0) {
                    const uint32_t v = lane < (uint32_t)kSeqWgClasses ? lhist[lane] : 0u;
                    uint32_t incl = v;
#pragma unroll
                    for (int o = 1; o < kWave; o <<= 1) {
                        const uint32_t y = __shfl_up(incl, o, kWave);
                        if ((int)lane >= o) incl += y;
                    }
                    if (lane < (uint32_t)kSeqWgClasses) lhist[lane] = incl - v;
                }
                __syncthreads();
                // cur[pos] = the row at walk position pos (until the starts replace it)
                for (uint32_t r = tid; r < sub_rows; r += kSeqWgThreads) cur[atomicAdd(&lhist[row_class(r)], 1u)] = r;
                __syncthreads();
            }
            uint32_t prow[kRowPasses], pv[kRowPasses];
#pragma unroll
            for (int u = 0; u < kRowPasses; u++) {
                const uint32_t pos = u * kSeqWgThreads + tid;
                prow[u] = pos < sub_rows ? (quad ? cur[pos] : pos) : 0u;
                pv[u] = pos < sub_rows ? (cnt[prow[u]] + kQuadStep - 1u) & ~(kQuadStep - 1u) : 0u;  // whole turns
            }
            __syncthreads();  // every row and count read before cur and cnt are rewritten
            uint32_t carry = 0;
#pragma unroll
            for (int u = 0; u < kRowPasses; u++) {
                if ((uint32_t)u * kSeqWgThreads >= sub_rows) break;  // uniform
                const uint32_t pos = u * kSeqWgThreads + tid;
                const uint32_t v = pv[u];
                uint32_t incl = v;
#pragma unroll
                for (int o = 1; o < kWave; o <<= 1) {
                    const uint32_t y = __shfl_up(incl, o, kWave);
                    if ((int)lane >= o) incl += y;
                }
                if (lane == kWave - 1) wsum[wave] = incl;
                __syncthreads();
                uint32_t wprefix = 0;
                for (uint32_t w = 0; w < wave; w++) wprefix += wsum[w];
                uint32_t total = 0;
                for (uint32_t w = 0; w < kSeqWgThreads / kWave; w++) total += wsum[w];
                const uint32_t start = carry + wprefix + incl - v;
                if (pos < sub_rows) {
                    cur[prow[u]] = start;
                    if (quad) cnt[pos] = prow[u] | (start / kQuadStep) << 12;
                }
                carry += total;
                __syncthreads();
            }
            if (quad && tid == 0) cnt[sub_rows] = (carry / kQuadStep) << 12;
            // scatter the entries' item numbers into their rows' buckets
            for (uint32_t it = wave; it < nb; it += kSeqWgThreads / kWave) {
                const uint32_t r = bitems[it];
                const uint32_t j = r % seq;
                const uint16_t *kt = ktab + (r / seq - r0 / seq) * seq;
                for (uint32_t i = lane; i < j; i += kWave) {
                    const uint32_t row = (((uint32_t)kt[i] << pe_dim) | ptab[j - i - 1]) & (sub_rows - 1);
                    ent[atomicAdd(&cur[row], 1u)] = (uint8_t)it;  // the item's gv row is it * cols
                }
            }
            // The quad path's gradient rows of a slice: thread tid loads columns
            // col0 + 4 (tid & 15) .. + 3 of items (tid >> 4) + 64 u, one slice
            // ahead (the loads run while the previous slice is walked); item nb
            // is the zero row.
            constexpr int kGvPasses = (kSeqWgGvWords / 64 + 63) / 64;
            u32x4 pre[kGvPasses];
            auto gv_load = [&](uint32_t col0) {
                const uint32_t cq = col0 + (tid & 15u) * 4u;
#pragma unroll
                for (int u = 0; u < kGvPasses; u++) {
                    const uint32_t it = (tid >> 4) + 64u * u;
                    pre[u] = u32x4{0u, 0u, 0u, 0u};
                    if (it < nb && cq < n_outputs)
                        pre[u] = *reinterpret_cast<const u32x4 *>(cv + (size_t)bitems[it] * n_outputs + cq);
                }
            };
            auto gv_store = [&]() {
#pragma unroll
                for (int u = 0; u < kGvPasses; u++) {
                    const uint32_t it = (tid >> 4) + 64u * u;
                    if (it <= nb) *reinterpret_cast<u32x4 *>(gv + it * 64u + (tid & 15u) * 4u) = pre[u];
                }
            };
            if (quad && !WIDE) gv_load(0);
            // The wide walk's pass of 128 columns: both planes' loads in flight
            // before their stores; the first pass's loads are issued here, to
            // land while the buckets are padded, a later pass's at the end of the
            // pass before
            u32x4 wlo[kGvPasses], whi[kGvPasses];
            auto wide_load = [&](uint32_t col0) {
                const uint32_t cq = col0 + (tid & 15u) * 4u;
#pragma unroll
                for (int u = 0; u < kGvPasses; u++) {
                    const uint32_t it = (tid >> 4) + 64u * u;
                    wlo[u] = u32x4{0u, 0u, 0u, 0u};
                    whi[u] = u32x4{0u, 0u, 0u, 0u};
                    if (it < nb) {
                        const uint32_t *src = cv + (size_t)bitems[it] * n_outputs + cq;
                        if (cq < n_outputs) wlo[u] = *reinterpret_cast<const u32x4 *>(src);
                        if (cq + 64u < n_outputs) whi[u] = *reinterpret_cast<const u32x4 *>(src + 64);
                    }
                }
            };
            if (WIDE) wide_load(0);
            // cur[row] is now the end of the row's entries.  The quad path pads
            // each bucket to whole turns with the zero row (item nb), and the two
            // words past the last turn too (the walk's read-ahead)
            if (quad) {
                __syncthreads();
                for (uint32_t r = tid; r < sub_rows; r += kSeqWgThreads)
                    for (uint32_t k = cur[r]; k & (kQuadStep - 1u); k++) ent[k] = (uint8_t)nb;
                if (tid < 2u * kQuadStep) ent[carry + tid] = (uint8_t)nb;
            }
            // the wide walk takes two 64-column slices a pass
            const uint32_t n_pass = WIDE ? (n_slices + 1) / 2 : n_slices;
            for (uint32_t sl = 0; sl < n_pass; sl++) {
                const uint32_t col0 = sl * cols * (WIDE ? 2u : 1u);
                __syncthreads();  // scatter done / the previous slice is done with gv
                // the batch's gradient rows, then a zero row (item nb) that the
                // quad path reads for pads
                if (WIDE) {
#pragma unroll
                    for (int u = 0; u < kGvPasses; u++) {
                        const uint32_t it = (tid >> 4) + 64u * u;
                        if (it <= nb) {
                            *reinterpret_cast<u32x4 *>(gv + it * 64u + (tid & 15u) * 4u) = wlo[u];
                            *reinterpret_cast<u32x4 *>(gv_hi + it * 64u + (tid & 15u) * 4u) = whi[u];
                        }
                        // dead until the next pass loads them: constants, so the
                        // walk holds no registers for them
                        wlo[u] = u32x4{0u, 0u, 0u, 0u};
                        whi[u] = u32x4{0u, 0u, 0u, 0u};
                    }
                } else if (quad) {
                    gv_store();
                } else {
                    for (uint32_t e = tid; e < (nb + 1) * cols; e += kSeqWgThreads) {
                        const uint32_t it = e / cols, cc = col0 + e % cols;
                        gv[e] = (it < nb && cc < n_outputs) ? cv[(size_t)bitems[it] * n_outputs + cc] : 0u;
                    }
                }
                __syncthreads();
                if (quad && !WIDE && sl + 1 < n_slices) gv_load(col0 + cols);
                const bool store = first && OVERWRITE;
                if (quad) {
                    // 64-column slices, lane k of a group holding columns 4k .. 4k+3:
                    // one 16-byte LDS read per entry.  Wavefront w takes walk
                    // positions 4 (w + 16 m) .. + 3, one per group, and adds four
                    // entries (one u32 of item numbers) a turn, the next turn's
                    // rows loading while this turn's are added (pads read the zero
                    // row, adding +0, which leaves a sum that starts at +0
                    // unchanged); the group then writes its row.  An entry's LDS
                    // address is item * 256 + the lane's byte offset (< 256): one
                    // byte permute builds it.
                    static_assert(kQuadStep == 4, "the walk reads entry quads");
                    const uint32_t c4 = (tid & 15u) * 4u;
                    const uint32_t cq = col0 + c4;
                    const uint32_t gw = (tid >> 4) & 3u;
                    const uint32_t lane_b = c4 * 4u;
                    const uint32_t *ent4 = reinterpret_cast<const uint32_t *>(ent);
                    const uint8_t *gvb = reinterpret_cast<const uint8_t *>(gv);
                    for (uint32_t k4 = wave * 4u; k4 < sub_rows; k4 += kSeqWgThreads / 16u) {
                        const uint32_t pos = k4 + gw;
                        const bool have = pos < sub_rows;
                        const uint32_t ps = min(pos, sub_rows - 1u);
                        const uint32_t w0 = cnt[ps], w1 = cnt[ps + 1u];
                        const uint32_t row = w0 & 0xFFFu;
                        const uint32_t e0q = w0 >> 12;
                        const uint32_t np = have ? (w1 >> 12) - e0q : 0u;  // turns
                        if constexpr (WIDE) {
                            // a pass of 128 columns: the same LDS offset in both
                            // 64-column planes, so one permute serves two reads
                            const uint8_t *gvh = reinterpret_cast<const uint8_t *>(gv_hi);
                            float af[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                            uint32_t ai[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
                            uint32_t pn = ent4[e0q];
                            for (uint32_t k = 0; k < np; k++) {
                                const uint32_t p2 = ent4[e0q + k + 1u];  // the next turn's entries
                                u32x4 gg[8];
#pragma unroll
                                for (int u = 0; u < 4; u++) {
                                    const uint32_t a = __builtin_amdgcn_perm(pn, lane_b, 0x0C0C0000u | ((4u + u) << 8));
                                    gg[u] = *reinterpret_cast<const u32x4 *>(gvb + a);
                                    gg[u + 4] = *reinterpret_cast<const u32x4 *>(gvh + a);
                                }
#pragma unroll
                                for (int u = 0; u < 4; u++)
#pragma unroll
                                    for (int c = 0; c < 4; c++) {
                                        if (INT_MODE) {
                                            ai[c] += gg[u][c];
                                            ai[c + 4] += gg[u + 4][c];
                                        } else {
                                            af[c] += __uint_as_float(gg[u][c]);
                                            af[c + 4] += __uint_as_float(gg[u + 4][c]);
                                        }
                                    }
                                pn = p2;
                            }
                            if (have && (store || np > 0)) {
#pragma unroll
                                for (int h = 0; h < 2; h++) {
                                    if (cq + 64u * h >= n_outputs) continue;
                                    u32x4 *p = reinterpret_cast<u32x4 *>(dst + (size_t)row * n_outputs + cq + 64u * h);
                                    u32x4 o;
                                    if (store) {
#pragma unroll
                                        for (int c = 0; c < 4; c++)
                                            o[c] = INT_MODE ? ai[4 * h + c] : __float_as_uint(af[4 * h + c]);
                                    } else {
                                        const u32x4 old = *p;
#pragma unroll
                                        for (int c = 0; c < 4; c++)
                                            o[c] = INT_MODE ? (uint32_t)wrap_add((int32_t)ai[4 * h + c], (int32_t)old[c])
                                                            : __float_as_uint(__uint_as_float(old[c]) + af[4 * h + c]);
                                    }
                                    *p = o;
                                }
                            }
                            continue;
                        }
                        float af[4] = {0.f, 0.f, 0.f, 0.f};
                        uint32_t ai[4] = {0u, 0u, 0u, 0u};
                        u32x4 ga[4], gb[4];
                        auto rows = [&](u32x4 (&gg)[4], uint32_t pr) {
#pragma unroll
                            for (int u = 0; u < 4; u++)
                                gg[u] = *reinterpret_cast<const u32x4 *>(
                                    gvb + __builtin_amdgcn_perm(pr, lane_b, 0x0C0C0000u | ((4u + u) << 8)));
                        };
                        auto add = [&](const u32x4 (&gg)[4]) {
#pragma unroll
                            for (int u = 0; u < 4; u++)
#pragma unroll
                                for (int c = 0; c < 4; c++) {
                                    if (INT_MODE) ai[c] += gg[u][c];
                                    else af[c] += __uint_as_float(gg[u][c]);
                                }
                        };
                        uint32_t pn = ent4[e0q + 1u];
                        rows(ga, ent4[e0q]);
                        for (uint32_t k = 0; k < np; k += 2) {
                            const uint32_t p2 = ent4[e0q + k + 2u];
                            rows(gb, pn);
                            add(ga);
                            if (k + 1u >= np) break;
                            pn = ent4[e0q + k + 3u];
                            rows(ga, p2);
                            add(gb);
                        }
                        if (have && (store || np > 0) && cq < n_outputs) {
                            u32x4 *p = reinterpret_cast<u32x4 *>(dst + (size_t)row * n_outputs + cq);
                            u32x4 o;
                            if (store) {
#pragma unroll
                                for (int c = 0; c < 4; c++) o[c] = INT_MODE ? ai[c] : __float_as_uint(af[c]);
                            } else {
                                const u32x4 old = *p;
#pragma unroll
                                for (int c = 0; c < 4; c++)
                                    o[c] = INT_MODE ? (uint32_t)wrap_add((int32_t)ai[c], (int32_t)old[c])
                                                    : __float_as_uint(__uint_as_float(old[c]) + af[c]);
                            }
                            *p = o;
                        }
                    }
                    // the wide walk's next pass: each wave issues its share of the
                    // loads once its rows are done, to land while others walk
                    if (WIDE && sl + 1 < n_pass) wide_load(col0 + 2 * cols);
                    continue;
                }
                // lane group g (cols lanes) takes the rows whose entries start in
                // [g E / G, (g + 1) E / G): about equal work whatever the row sizes
                const uint32_t lanes = cols;
                const uint32_t n_groups = kSeqWgThreads / lanes, grp = tid / lanes;
                const uint32_t total = cur[sub_rows - 1];  // entries of the batch
                auto first_row = [&](uint32_t gi) -> uint32_t {
                    if (gi >= n_groups) return sub_rows;
                    const uint32_t tgt = (uint32_t)(((uint64_t)total * gi + n_groups - 1) / n_groups);
                    uint32_t lo = 0, hi = sub_rows;  // first row r with start(r) >= tgt
                    while (lo < hi) {
                        const uint32_t mid = (lo + hi) / 2;
                        if (cur[mid] - cnt[mid] < tgt) lo = mid + 1; else hi = mid;
                    }
                    return gi == 0 ? 0u : lo;
                };
                const uint32_t rs = first_row(grp), re = first_row(grp + 1);
                const uint32_t cc = col0 + my_col;
                for (uint32_t row = rs; row < re; row++) {
                    const uint32_t e1 = cur[row];
                    uint32_t e = e1 - cnt[row];
                    // a row without entries in this batch keeps what it holds
                    // (it is only written when this pass stores)
                    if (!store && e == e1) continue;
                    uint32_t a = 0u;
                    // eight entries at a time, their LDS reads in flight together;
                    // the last group re-reads the row's last entry and adds +0
                    // past its end (the sum starts at +0 and is never -0, so
                    // that changes nothing)
                    for (; e < e1; e += 8) {
                        uint32_t v[8];
#pragma unroll
                        for (int u = 0; u < 8; u++) {
                            const uint32_t g = gv[(uint32_t)ent[min(e + u, e1 - 1)] * cols + my_col];
                            v[u] = e + u < e1 ? g : 0u;
                        }
                        if (INT_MODE) {
#pragma unroll
                            for (int u = 0; u < 8; u++) a += v[u];
                        } else {
                            float f = __uint_as_float(a);
#pragma unroll
                            for (int u = 0; u < 8; u++) f += __uint_as_float(v[u]);
                            a = __float_as_uint(f);
                        }
                    }
                    // this batch's sum of (row, cc): rows q * sub_rows .. of table t
                    if (cc < n_outputs) {
                        float *p = dst + (size_t)row * n_outputs + cc;
                        float v;
                        if (INT_MODE) {
                            int32_t iv = (int32_t)a;
                            if (!store) iv = wrap_add(iv, __float_as_int(*p));
                            // the int epilogue runs after the last batch; until
                            // then the sums stay int32 bits
                            v = __int_as_float(iv);
                        } else {
                            v = __uint_as_float(a);
                            if (!store) v = *p + v;
                        }
                        *p = v;
                    }
                }
            }
            first = false;
        }
        k0 = k1;
    }
    if (INT_MODE) {
        // int epilogue of the sub-table (every row; untouched ones hold the
        // caller's int bits or, when overwriting, zero)
        __syncthreads();
        for (uint32_t e = tid; e < sub_rows * n_outputs; e += kSeqWgThreads) {
            float *p = dst + e;
            const int32_t iv = (first && OVERWRITE) ? 0 : __float_as_int(*p);
            *p = (float)(((double)iv * kDenom32Reciproc) / int_rescaler);
        }
    } else if (first && OVERWRITE) {
        // an empty bucket: its sub-table gradient is zero
        for (uint32_t e = tid; e < sub_rows * n_outputs; e += kSeqWgThreads) dst[e] = 0.0f;
    }
}

// Fallback weight gradient: one thread per (b, t, j, output) with global atomics.
template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_wgrad_seq_atomic(
    const uint32_t *__restrict__ cv, const uint2 *__restrict__ pack, const uint2 *__restrict__ ppack,
    float *__restrict__ target, uint32_t batch, uint32_t seq, uint32_t n_outputs,
    uint32_t n_detectors, uint32_t n_anchors, uint32_t pe_dim, uint64_t n_items) {
    const uint64_t it = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    if (it >= n_items) return;
    const uint32_t o = (uint32_t)(it % n_outputs);
    const uint64_t r = it / n_outputs;
    const uint32_t j = (uint32_t)(r % seq);
    const uint32_t t = (uint32_t)((r / seq) % n_detectors);
    const uint32_t b = (uint32_t)(r / ((uint64_t)seq * n_detectors));
    const uint32_t n_rows = batch * seq;
    const uint32_t kbits = n_anchors + pe_dim;
    const uint32_t pmask = (1u << pe_dim) - 1;
    const uint2 *kp = pack + (size_t)t * n_rows + (size_t)b * seq;
    const uint32_t Q = rec_idx(kp[j]);
    const uint32_t v = cv[((size_t)b * seq + j) * n_outputs + o];
    float *wt = target + (size_t)t * (1u << (n_anchors + kbits)) * n_outputs;
    for (uint32_t i = 0; i < j; i++) {
        const uint32_t row = (Q << kbits) | (rec_idx(kp[i]) << pe_dim) |
                             (rec_idx(ppack[(size_t)t * (seq - 1) + (j - i - 1)]) & pmask);
        float *p = wt + (size_t)row * n_outputs + o;
        if (INT_MODE)
            atomicAdd(reinterpret_cast<int32_t *>(p), (int32_t)v);
        else
            unsafeAtomicAdd(p, __uint_as_float(v));
    }
}

uint32_t blocks_for(uint64_t n) { return (uint32_t)((n + kBlock - 1) / kBlock); }

uint32_t seq_vec(uint32_t n_outputs) {
    if (n_outputs % 4 == 0 && n_outputs >= 64u * 4u * 4u) return 4;
    if (n_outputs % 2 == 0 && n_outputs >= 64u * 2u * 4u) return 2;
    return 1;
}

// Bytes of one pair triangle [B][T][S(S-1)/2] of fp64.
uint64_t seq_tri_bytes(const SeqShape &s) {
    return (uint64_t)s.batch * s.n_detectors * ((uint64_t)s.seq * (s.seq - 1) / 2) * 8;
}

// The pair-parallel main pass and its triangle reduction apply (fp32 sums).
bool seq_pairs_applies(const SeqShape &s) {
    return s.n_outputs % 4 == 0 && s.n_outputs <= (uint32_t)kPairMaxO && seq_tri_bytes(s) <= (16ull << 30);
}

// K-group bits of the grouped input-gradient pass (-1: it does not apply):
// the widest group whose 2^(gb + Npe) rows fit the 128 KiB LDS table.
int seq_grp_bits(const SeqShape &s) {
    if (s.n_outputs != 64 && s.n_outputs != 128 && s.n_outputs != 256) return -1;
    if (s.n_anchors > 10 || s.seq < 2 || s.seq - 1 > (uint32_t)kGrpMaxDist) return -1;
    if ((uint64_t)s.batch * s.seq >= (1ull << 27)) return -1;  // rows in 27 bits of the item metadata
    uint32_t lr = 0;
    while ((kGrpTabBytes >> (lr + 1)) >= (int)(s.n_outputs * 4)) lr++;
    if (s.pe_dim > lr) return -1;
    return (int)std::min<uint32_t>(s.n_anchors, lr - s.pe_dim);
}

// Columns of a forward slice for k_fill_seq_lds (0: it does not apply): the
// widest power of two <= 64 whose sub-table slice fits the LDS table.
uint32_t seq_fill_cols(const SeqShape &s) {
    const uint64_t sub_rows = 1ull << (s.n_anchors + s.pe_dim);
    const uint64_t rows = (uint64_t)s.batch * s.seq;
    if (s.n_outputs % 4 != 0 || s.seq - 1 > (uint32_t)kSfPe || rows > 0x7fffffffull ||
        (uint64_t)s.n_detectors * rows * s.n_outputs * 4 > (8ull << 30))
        return 0;
    uint32_t cols = 64;
    while (cols > 8 && sub_rows * cols > (uint64_t)kSfTabFloats) cols /= 2;
    if (sub_rows * cols > (uint64_t)kSfTabFloats) return 0;
    while (cols > 8 && cols / 2 >= s.n_outputs) cols /= 2;
    return cols;
}

// Columns of a weight-gradient slice (0: the sort path does not apply): a
// power of two <= 64 (one lane per column of a lane group).
uint32_t seq_wg_cols(const SeqShape &s) {
    const uint64_t sub_rows = 1ull << (s.n_anchors + s.pe_dim);
    if (sub_rows > (uint64_t)kSeqWgRowsMax || s.seq > (uint32_t)kSeqWgKeys ||
        s.seq - 1 > (uint32_t)kSeqWgPe || s.seq - 1 + (kQuadStep - 1) * sub_rows > (uint64_t)kSeqWgEntries)
        return 0;
    uint32_t cols = 64;
    while (cols > 1 && cols / 2 >= s.n_outputs) cols /= 2;
    return cols;
}

// Items per batch: their entries (< seq each) and gradient rows must fit.
uint32_t seq_wg_items(const SeqShape &s, uint32_t cols) {
    const uint32_t sub_rows = 1u << (s.n_anchors + s.pe_dim);
    uint32_t n = ((uint32_t)kSeqWgEntries - (kQuadStep - 1) * sub_rows) / std::max<uint32_t>(1, s.seq - 1);  // and pads
    n = std::min<uint32_t>(n, (uint32_t)kSeqWgGvWords / cols - 1);  // and the zero row
    return std::min<uint32_t>(n, (uint32_t)kSeqWgItems);
}

}  // namespace

hipError_t launch_seq_indices(const SeqShape &s, const float *x, const int32_t *anchors,
                              const float *pe, int32_t *idx, int32_t *pidx, float *md, int32_t *mi,
                              float *pmd, int32_t *pmi, float cmp_eps, hipStream_t st) {
    FcShape fs{};
    fs.batch = s.batch * s.seq;
    fs.n_inputs = s.n_inputs;
    fs.n_outputs = s.n_outputs;
    fs.n_detectors = s.n_detectors;
    fs.n_anchors = s.n_anchors;
    fs.n_entries = 1u << s.n_anchors;
    fs.dgs = s.dgs;
    fs.ogs = s.ogs;
    hipError_t e = launch_check_detectors(fs, x, anchors, cmp_eps, idx, md, mi, st);
    if (e != hipSuccess) return e;
    const uint32_t n_pe = (s.seq - 1) * s.n_detectors;
    if (s.pe_dim > 0 && n_pe > 0) {
        if (md)
            hipLaunchKernelGGL(k_check_pe<true>, dim3(blocks_for(n_pe)), dim3(kBlock), 0, st, pe,
                               n_pe, s.pe_dim, cmp_eps, pidx, pmd, pmi);
        else
            hipLaunchKernelGGL(k_check_pe<false>, dim3(blocks_for(n_pe)), dim3(kBlock), 0, st, pe,
                               n_pe, s.pe_dim, cmp_eps, pidx, (float *)nullptr, (int32_t *)nullptr);
        e = hipGetLastError();
    }
    return e;
}

hipError_t launch_forward_seq(const SeqShape &s, const float *w, const float *x,
                              const int32_t *anchors, const float *pe, float *out, int32_t *idx,
                              int32_t *pidx, float *md, int32_t *mi, float *pmd, int32_t *pmi,
                              float cmp_eps, bool int_mode, double int_rescaler, Scratch &scratch,
                              hipStream_t st) {
    const uint32_t rows = s.batch * s.seq;
    const uint32_t fcols = seq_fill_cols(s);
    // scratch: packed keys [T][B*S] | positional keys [T][S-1] | and for the
    // LDS-sliced forward: bucket offsets [T][2^Nc+1] | samples [T][B*S] |
    // per-table partials [T][B*S][O]
    ScratchLayout lay(scratch);
    uint2 *pack = lay.take<uint2>((size_t)rows * s.n_detectors * 8);
    uint2 *ppack = lay.take<uint2>((size_t)s.n_detectors * (s.seq - 1) * 8);
    int32_t *offsets = nullptr, *samples = nullptr;
    uint32_t *part = nullptr, *order = nullptr;
    if (fcols > 0) {
        offsets = lay.take<int32_t>((size_t)s.n_detectors * ((1u << s.n_anchors) + 1) * 4);
        samples = lay.take<int32_t>((size_t)s.n_detectors * rows * 4);
        part = lay.take<uint32_t>((size_t)s.n_detectors * rows * s.n_outputs * 4);
        order = lay.take<uint32_t>((size_t)s.n_detectors * (1u << s.n_anchors) * 4);
    }
    hipError_t e;
    if (lay.stop(&e, "forward_step_concat")) return e;
    FcShape fs{};
    fs.batch = rows;
    fs.n_inputs = s.n_inputs;
    fs.n_outputs = s.n_outputs;
    fs.n_detectors = s.n_detectors;
    fs.n_anchors = s.n_anchors;
    fs.n_entries = 1u << s.n_anchors;
    fs.dgs = s.dgs;
    fs.ogs = s.ogs;
    e = launch_seq_indices(s, x, anchors, pe, idx, pidx, md, mi, pmd, pmi, cmp_eps, st);
    if (e != hipSuccess) return e;
    const uint32_t n_pe = (s.seq - 1) * s.n_detectors;
    hipLaunchKernelGGL(k_seq_pack, dim3((s.n_detectors + 63) / 64, (rows + 63) / 64), dim3(kBlock),
                       0, st, idx, (const float *)nullptr, (const int32_t *)nullptr, pack, rows,
                       s.n_detectors);
    hipLaunchKernelGGL(k_seq_pack_pe, dim3(blocks_for(n_pe)), dim3(kBlock), 0, st,
                       s.pe_dim > 0 ? pidx : (const int32_t *)nullptr, (const float *)nullptr,
                       (const int32_t *)nullptr, ppack, s.seq - 1, s.n_detectors);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (fcols > 0) {
        FcShape fs2 = fs;
        e = launch_bucket_samples(fs2, idx, offsets, samples, st);
        if (e != hipSuccess) return e;
        const uint32_t n_slices = (s.n_outputs + fcols - 1) / fcols;
        const uint64_t grid = (uint64_t)s.n_detectors * (1u << s.n_anchors) * n_slices;
        if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
        // workgroups take the buckets largest first (an input with few distinct
        // rows, such as a token embedding, concentrates its Q values)
        const uint32_t n_buckets = s.n_detectors * (1u << s.n_anchors);
        if (n_buckets <= kOrderMaxBuckets)
            hipLaunchKernelGGL(k_bucket_order, dim3(1), dim3(kSeqWgThreads), 0, st, offsets,
                               1u << s.n_anchors, n_buckets, order);
        else
            order = nullptr;
#define SPIKY_FLDS(C, IM)                                                                          \
    hipLaunchKernelGGL((k_fill_seq_lds<C, IM>), dim3((uint32_t)grid), dim3(kSfThreads), 0, st, w,    \
                       pack, ppack, offsets, samples, order, part, s.batch, s.seq, s.n_outputs,     \
                       s.n_anchors, s.pe_dim, n_slices, int_rescaler)
        switch (fcols) {
            case 64: if (int_mode) SPIKY_FLDS(64, true); else SPIKY_FLDS(64, false); break;
            case 32: if (int_mode) SPIKY_FLDS(32, true); else SPIKY_FLDS(32, false); break;
            case 16: if (int_mode) SPIKY_FLDS(16, true); else SPIKY_FLDS(16, false); break;
            default: if (int_mode) SPIKY_FLDS(8, true); else SPIKY_FLDS(8, false); break;
        }
#undef SPIKY_FLDS
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_block_commit(part, out, (uint64_t)rows * s.n_outputs, s.n_detectors, int_mode,
                                   int_rescaler, st);
    }
    const uint32_t vec = seq_vec(s.n_outputs);
    const uint32_t n_slices = (s.n_outputs + kWave * vec - 1) / (kWave * vec);
    const uint64_t units = (uint64_t)s.batch * (s.seq - 1);
    const uint64_t grid = (uint64_t)n_slices * ((units + kWPB - 1) / kWPB);
    if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
#define SPIKY_FSEQ(V, IM)                                                                         \
    hipLaunchKernelGGL((k_fill_seq<V, IM>), dim3((uint32_t)grid), dim3(kBlock), 0, st, w, pack,    \
                       ppack, out, s.batch, s.seq, s.n_outputs, s.n_detectors, s.n_anchors,        \
                       s.pe_dim, n_slices, int_rescaler)
    switch (vec) {
        case 4: if (int_mode) SPIKY_FSEQ(4, true); else SPIKY_FSEQ(4, false); break;
        case 2: if (int_mode) SPIKY_FSEQ(2, true); else SPIKY_FSEQ(2, false); break;
        default: if (int_mode) SPIKY_FSEQ(1, true); else SPIKY_FSEQ(1, false); break;
    }
#undef SPIKY_FSEQ
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // position 0 has no earlier token; in int mode its int32 accumulator still
    // needs the epilogue
    if (int_mode) {
        for (uint32_t b = 0; b < s.batch; b++) {
            e = launch_convert_i2f(out + (size_t)b * s.seq * s.n_outputs, s.n_outputs, int_rescaler, st);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

hipError_t launch_backward_seq(const SeqShape &s, float *w, const float *g, const int32_t *anchors,
                               const int32_t *idx, const float *md, const int32_t *mi,
                               const int32_t *pidx, const float *pmd, const int32_t *pmi,
                               float *x_grad, float *pe_grad, float *target, double lr,
                               bool overwrite, bool int_mode, double int_rescaler, Scratch &scratch,
                               hipStream_t st) {
    const uint32_t rows = s.batch * s.seq;
    const uint32_t n_pe = (s.seq - 1) * s.n_detectors;
    const size_t n_dpe = (size_t)n_pe * std::max<uint32_t>(s.pe_dim, 1);
    const int gb = int_mode ? -1 : seq_grp_bits(s);
    const bool pairs = gb < 0 && seq_pairs_applies(s);
    // scratch: packed keys [T][B*S] | positional keys [T][S-1] | dq, dq_alt,
    // dk [B*S][T] f64 | dpe [(S-1)][T][Npe] f64 | bucket offsets [T][2^Nc+1] |
    // samples [T][B*S] | commit values [B*S][O] | Q-flipped keys [B*S][T] |
    // their bucket offsets [T][2^(Nc+1)+1] and samples [T][B*S] | then the
    // pair triangles of the pair-parallel pass, or the position lists of the
    // grouped pass
    ScratchLayout lay(scratch);
    uint2 *pack = lay.take<uint2>((size_t)rows * s.n_detectors * 8);
    uint2 *ppack = lay.take<uint2>((size_t)s.n_detectors * (s.seq - 1) * 8);
    double *dq = lay.take<double>((size_t)rows * s.n_detectors * 8);
    double *dq_alt = lay.take<double>((size_t)rows * s.n_detectors * 8);
    double *dk = lay.take<double>((size_t)rows * s.n_detectors * 8);
    double *dpe = lay.take<double>(n_dpe * 8);
    int32_t *offsets = lay.take<int32_t>((size_t)s.n_detectors * ((1u << s.n_anchors) + 1) * 4);
    int32_t *samples = lay.take<int32_t>((size_t)s.n_detectors * rows * 4);
    uint32_t *cv = lay.take<uint32_t>((size_t)rows * s.n_outputs * 4);
    int32_t *alt_keys = lay.take<int32_t>((size_t)rows * s.n_detectors * 4);
    int32_t *offsets2 = lay.take<int32_t>((size_t)s.n_detectors * ((2u << s.n_anchors) + 1) * 4);
    int32_t *samples2 = lay.take<int32_t>((size_t)s.n_detectors * rows * 4);
    double *tk = pairs ? lay.take<double>(seq_tri_bytes(s)) : nullptr;
    double *tp = pairs ? lay.take<double>(seq_tri_bytes(s)) : nullptr;
    uint32_t *wg_order = lay.take<uint32_t>((size_t)s.n_detectors * (1u << s.n_anchors) * 4);
    uint2 *list_a = nullptr, *list_b = nullptr;
    uint32_t *off_a = nullptr, *off_b = nullptr;
    if (gb >= 0) {
        const uint64_t tb = (uint64_t)s.n_detectors * s.batch;
        const uint64_t ng = 1ull << (s.n_anchors - gb);
        list_a = lay.take<uint2>(tb * s.seq * 8);
        list_b = lay.take<uint2>(tb * s.seq * 8);
        off_a = lay.take<uint32_t>(tb * (ng + 1) * 4);
        off_b = lay.take<uint32_t>(tb * (ng + 1) * 4);
    }
    hipError_t e;
    if (lay.stop(&e, "backward_backprop_concat")) return e;

    hipLaunchKernelGGL(k_seq_pack, dim3((s.n_detectors + 63) / 64, (rows + 63) / 64), dim3(kBlock),
                       0, st, idx, md, mi, pack, rows, s.n_detectors);
    hipLaunchKernelGGL(k_seq_pack_pe, dim3(blocks_for(n_pe)), dim3(kBlock), 0, st,
                       s.pe_dim > 0 ? pidx : (const int32_t *)nullptr, pmd, pmi, ppack, s.seq - 1,
                       s.n_detectors);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int2 *ap = reinterpret_cast<const int2 *>(anchors);

    FcShape fs{};
    fs.batch = rows;
    fs.n_inputs = s.n_inputs;
    fs.n_outputs = s.n_outputs;
    fs.n_detectors = s.n_detectors;
    fs.n_anchors = s.n_anchors;
    fs.n_entries = 1u << s.n_anchors;
    fs.dgs = s.dgs;
    fs.ogs = s.ogs;
    // (t, Q) buckets of the rows: the propagate's schedule and the weight
    // gradient's sub-tables
    e = launch_bucket_samples(fs, idx, offsets, samples, st);
    if (e != hipSuccess) return e;

    // input and positional gradients
    const uint32_t nj = (s.n_outputs + 255) / 256;
    if (!int_mode && s.n_outputs % 4 == 0 && nj <= 4) {
        const uint64_t n_acc = (uint64_t)rows * s.n_detectors;
        hipLaunchKernelGGL(k_zero64, dim3(blocks_for(n_acc)), dim3(kBlock), 0, st, dq, n_acc);
        hipLaunchKernelGGL(k_zero64, dim3(blocks_for(n_acc)), dim3(kBlock), 0, st, dq_alt, n_acc);
        hipLaunchKernelGGL(k_zero64, dim3(blocks_for(n_acc)), dim3(kBlock), 0, st, dk, n_acc);
        hipLaunchKernelGGL(k_seq_alt_keys, dim3(blocks_for(n_acc)), dim3(kBlock), 0, st, idx, mi,
                           alt_keys, n_acc, s.n_anchors);
        FcShape fs_alt = fs;
        fs_alt.n_entries = 2u << s.n_anchors;
        e = launch_bucket_samples(fs_alt, alt_keys, offsets2, samples2, st);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_zero64, dim3(blocks_for(n_dpe)), dim3(kBlock), 0, st, dpe, (uint64_t)n_dpe);
        const uint64_t units = (uint64_t)rows * s.n_detectors;  // one workgroup each
        const uint64_t wg_per_xcd = (units + 7) / 8;
        const uint64_t grid = wg_per_xcd * 8;
        if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
#define SPIKY_PSEQ(NJ, ALT, SMP, QS)                                                                 \
    hipLaunchKernelGGL((k_propagate_seq<NJ, ALT>), dim3((uint32_t)grid), dim3(kBlock), 0, st, w, g, \
                       pack, ppack, SMP, QS, dk, dpe, s.batch, s.seq, s.n_outputs, s.n_detectors,   \
                       s.n_anchors, s.pe_dim, (uint32_t)wg_per_xcd)
#define SPIKY_PSEQ2(NJ)                                \
    SPIKY_PSEQ(NJ, false, samples, dq);                \
    SPIKY_PSEQ(NJ, true, samples2, dq_alt)
        if (gb >= 0) {
            const uint32_t ng = 1u << (s.n_anchors - gb);
            hipLaunchKernelGGL(k_seq_group_lists, dim3(s.n_detectors * s.batch), dim3(kWave), 0, st,
                               pack, list_a, off_a, list_b, off_b, s.batch, s.seq, s.n_anchors,
                               (uint32_t)gb);
            const uint64_t n_wg = (uint64_t)s.n_detectors * (1u << s.n_anchors) * ng;
            const uint64_t per_xcd = (n_wg + 7) / 8;
            if (per_xcd * 8 > 0x7fffffffu) return hipErrorInvalidConfiguration;
#define SPIKY_PGRP(NCH)                                                                             \
    hipLaunchKernelGGL(k_propagate_seq_grp<NCH>, dim3((uint32_t)(per_xcd * 8)), dim3(kGrpThreads), \
                       0, st, w, g, pack, ppack, offsets, samples, offsets2, samples2, list_a,      \
                       off_a, list_b, off_b, dq, dpe, s.batch, s.seq, s.n_detectors, s.n_anchors,   \
                       s.pe_dim, (uint32_t)gb, (uint32_t)per_xcd)
            switch (s.n_outputs) {
                case 64: SPIKY_PGRP(2); break;
                case 128: SPIKY_PGRP(4); break;
                default: SPIKY_PGRP(8); break;
            }
#undef SPIKY_PGRP
            hipLaunchKernelGGL(k_seq_xgrad, dim3(blocks_for(n_acc)), dim3(kBlock), 0, st, dq,
                               (const double *)nullptr, (const double *)nullptr, pack, ap, x_grad,
                               s.batch, s.seq, s.n_inputs, s.n_detectors, s.n_anchors);
        } else if (pairs) {
            hipLaunchKernelGGL(k_propagate_seq_pairs, dim3((uint32_t)grid), dim3(kBlock),
                               pair_g_doubles(s.n_outputs) * sizeof(double), st, w, g,
                               pack, ppack, samples, dq, tk, tp, s.batch, s.seq, s.n_outputs,
                               s.n_detectors, s.n_anchors, s.pe_dim, (uint32_t)wg_per_xcd);
            switch (nj) {
                case 1: SPIKY_PSEQ(1, true, samples2, dq_alt); break;
                case 2: SPIKY_PSEQ(2, true, samples2, dq_alt); break;
                case 3: SPIKY_PSEQ(3, true, samples2, dq_alt); break;
                default: SPIKY_PSEQ(4, true, samples2, dq_alt); break;
            }
            hipLaunchKernelGGL(k_seq_tri_reduce, dim3(s.batch * s.n_detectors), dim3(kBlock), 0, st,
                               tk, tp, dq, dq_alt, pack, ppack, ap, x_grad, dpe, s.batch, s.seq,
                               s.n_inputs, s.n_detectors, s.n_anchors, s.pe_dim);
        } else {
            switch (nj) {
                case 1: SPIKY_PSEQ2(1); break;
                case 2: SPIKY_PSEQ2(2); break;
                case 3: SPIKY_PSEQ2(3); break;
                default: SPIKY_PSEQ2(4); break;
            }
            hipLaunchKernelGGL(k_seq_xgrad, dim3(blocks_for(n_acc)), dim3(kBlock), 0, st, dq, dq_alt,
                               dk, pack, ap, x_grad, s.batch, s.seq, s.n_inputs, s.n_detectors,
                               s.n_anchors);
        }
#undef SPIKY_PSEQ2
#undef SPIKY_PSEQ
        if (s.pe_dim > 0)
            hipLaunchKernelGGL(k_seq_pe_commit, dim3(blocks_for(n_dpe)), dim3(kBlock), 0, st, dpe,
                               pe_grad, (uint32_t)n_dpe);
    } else {
        const uint32_t n_ob = (s.n_outputs + s.ogs - 1) / s.ogs;
        const uint64_t n_items = (uint64_t)s.batch * s.n_detectors * ((uint64_t)s.seq * (s.seq - 1) / 2) * n_ob;
        if (n_items > 0) {
            if (n_items / kBlock > 0x7fffffffull) return hipErrorInvalidConfiguration;
            if (int_mode)
                hipLaunchKernelGGL(k_propagate_seq_exact<true>, dim3(blocks_for(n_items)), dim3(kBlock),
                                   0, st, w, g, pack, ppack, ap, x_grad, pe_grad, s.batch, s.seq,
                                   s.n_inputs, s.n_outputs, s.n_detectors, s.n_anchors, s.pe_dim,
                                   s.ogs, n_ob, n_items, int_rescaler);
            else
                hipLaunchKernelGGL(k_propagate_seq_exact<false>, dim3(blocks_for(n_items)),
                                   dim3(kBlock), 0, st, w, g, pack, ppack, ap, x_grad, pe_grad,
                                   s.batch, s.seq, s.n_inputs, s.n_outputs, s.n_detectors,
                                   s.n_anchors, s.pe_dim, s.ogs, n_ob, n_items, int_rescaler);
        }
        if (int_mode) {
            e = launch_convert_i2f(x_grad, (uint64_t)rows * s.n_inputs, int_rescaler, st);
            if (e != hipSuccess) return e;
            if (s.pe_dim > 0) {
                e = launch_convert_i2f(pe_grad, (uint64_t)n_pe * s.pe_dim, int_rescaler, st);
                if (e != hipSuccess) return e;
            }
        }
    }
    e = hipGetLastError();
    if (e != hipSuccess || target == nullptr) return e;

    // weight gradient (or the in-place update of the weights)
    e = launch_wgrad_commit_values(g, cv, (uint64_t)rows * s.n_outputs, lr, int_mode, int_rescaler, st);
    if (e != hipSuccess) return e;
    const uint32_t cols = seq_wg_cols(s);
    if (cols > 0) {
        const uint32_t n_slices = (s.n_outputs + cols - 1) / cols;
        const uint64_t grid = (uint64_t)s.n_detectors * (1u << s.n_anchors);
        if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
        const uint32_t ipb = seq_wg_items(s, cols);
        // 16-byte row pieces: 64-column slices of whole quads, 16-byte aligned rows
        const bool quad = cols == 64 && s.n_outputs % 4 == 0 && ((uintptr_t)target & 15) == 0;
        // two 64-column slices a pass where the sub-table's row arrays leave LDS room
        const bool wide = quad && (1u << (s.n_anchors + s.pe_dim)) <= (uint32_t)kSeqWgWideRows;
        if (grid <= kOrderMaxBuckets)
            hipLaunchKernelGGL(k_bucket_order, dim3(1), dim3(kSeqWgThreads), 0, st, offsets,
                               1u << s.n_anchors, (uint32_t)grid, wg_order);
        else
            wg_order = nullptr;
#define SPIKY_WSEQ(IM, OW, WD)                                                                              \
    hipLaunchKernelGGL((k_wgrad_seq_sort<IM, OW, WD>), dim3((uint32_t)grid), dim3(kSeqWgThreads), 0, st, cv, \
                       offsets, samples, pack, ppack, wg_order, target, s.batch, s.seq, s.n_outputs,        \
                       s.n_detectors, s.n_anchors, s.pe_dim, cols, n_slices, ipb, int_rescaler, quad)
#define SPIKY_WSEQ_W(IM, OW)           \
    if (wide)                          \
        SPIKY_WSEQ(IM, OW, true);      \
    else                               \
        SPIKY_WSEQ(IM, OW, false);
        if (int_mode) {
            if (overwrite) { SPIKY_WSEQ_W(true, true) } else { SPIKY_WSEQ_W(true, false) }
        } else {
            if (overwrite) { SPIKY_WSEQ_W(false, true) } else { SPIKY_WSEQ_W(false, false) }
        }
#undef SPIKY_WSEQ_W
#undef SPIKY_WSEQ
        return hipGetLastError();
    }
    const uint64_t n_w = (uint64_t)s.n_detectors * (1ull << (2 * s.n_anchors + s.pe_dim)) * s.n_outputs;
    if (overwrite) {
        e = launch_zero(target, n_w, st);
        if (e != hipSuccess) return e;
    }
    const uint64_t n_items = (uint64_t)rows * s.n_detectors * s.n_outputs;
    if (int_mode)
        hipLaunchKernelGGL(k_wgrad_seq_atomic<true>, dim3(blocks_for(n_items)), dim3(kBlock), 0, st,
                           cv, pack, ppack, target, s.batch, s.seq, s.n_outputs, s.n_detectors,
                           s.n_anchors, s.pe_dim, n_items);
    else
        hipLaunchKernelGGL(k_wgrad_seq_atomic<false>, dim3(blocks_for(n_items)), dim3(kBlock), 0, st,
                           cv, pack, ppack, target, s.batch, s.seq, s.n_outputs, s.n_detectors,
                           s.n_anchors, s.pe_dim, n_items);
    e = hipGetLastError();
    if (e != hipSuccess || !int_mode) return e;
    return launch_convert_i2f(target, n_w, int_rescaler, st);
}

}  // namespace spiky
