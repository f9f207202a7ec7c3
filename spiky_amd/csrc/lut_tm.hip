// lut_tm.hip -- table-major ("stage once, serve every sample") kernels for the
// fully connected LUT layer on gfx950.
//
// A work unit is (block of `dgs` tables, slice of 32 output columns, chunk of
// samples).  The unit streams its tables' 128-byte row chunks (all E rows of a
// table, 32 KiB at E = 256) from HBM into LDS exactly once, double-buffered
// through registers, and 1024 threads then serve every sample of the chunk
// from LDS.  Each table byte therefore crosses HBM once per sample chunk
// instead of once per sample that hits its row, which is what makes the
// gather compulsory-traffic bound.
//
// Thread layout inside a unit: wavefront w (0..15), lane l: sample
// w*8 + l/8 (+128*i for i < SPT), column quad l%8 (columns slice*32 + 4*(l%8)
// .. +3).  The 8 lanes of one sample read one 128-byte LDS row, so the read is
// free of bank conflicts.
//
// Forward: the unit writes, for every sample, the fp32 (or int32 fixed-point)
// commit value of its table block -- (float)(fp64 sum over the block's tables,
// ascending) -- into a partial buffer; k_fill_commit then adds the blocks in
// ascending order onto the output.  That is exactly the reference CPU path's
// arithmetic (lut_runtime_kernels_logic.proto:1214-1299 run serially,
// misc.h:119-129), so the output stays bit-identical to it.
//
// Propagate: the unit writes, for every (sample, table), the fp64 dot of its
// 32 columns, sum_c (W[main][c] - W[alt][c]) * g[c], rounded to fp32, into a
// partial buffer [slice][table][sample]; k_propagate_reduce sums the slices in
// a fixed order and scales by du(min margin) into du[sample][table], and
// k_propagate_scatter accumulates the input gradient of a few samples in LDS
// before adding it to HBM once (no global atomics).
#include "lut_kernels.h"

#include <algorithm>
#include <type_traits>

namespace spiky {
namespace {

constexpr int kWave = 64;
constexpr int kTmThreads = 1024;
constexpr int kTmCols = 32;
constexpr int kTmPass = (kTmThreads / kWave) * 8;  // samples per pass of SPT = 1
constexpr int kTmMaxEntries = 256;
constexpr int kTmPF = 2;  // tables per pipeline stage

// native vector types: they stay in registers across the staging loop, where
// HIP's struct-based float4 is demoted to scratch memory
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ double du_of_margin(float md) {
    double du = (double)md;
    double r = 1.0 / (1.0 + fabs(du));
    return (du > 0) ? r * (0.5 * r) : r * (-0.5 * r);
}

__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

// DPP lane exchange of an fp64 value (two 32-bit moves on the VALU).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double((long long)(((unsigned long long)(uint32_t)hi << 32) |
                                            (unsigned long long)(uint32_t)lo));
}
constexpr int kDppHalfMirror = 0x141;  // lane l of 8 <-> 7 - l
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]

// One reduce-scatter step over a lane pairing: the pair sums its N items and
// each lane keeps half of them (the lane with `upper` set keeps the upper
// half); with N == 1 both lanes keep the single sum.
template <int CTRL, int N>
__device__ __forceinline__ void rs_step(double (&v)[8], bool upper) {
    if (N == 1) {
        v[0] += dpp_f64<CTRL>(v[0]);
        return;
    }
    constexpr int M = N / 2;
#pragma unroll
    for (int j = 0; j < M; j++) {
        const double send = upper ? v[j] : v[M + j];
        const double keep = upper ? v[M + j] : v[j];
        v[j] = keep + dpp_f64<CTRL>(send);
    }
}

// Sums item j (< N) of the 8 lanes of every lane group; afterwards lane l of
// the group holds the sum of item rs_item<N>(l) in v[0], and rs_writer<N>(l)
// marks one lane per item.
template <int N>
__device__ __forceinline__ void reduce_scatter8(double (&v)[8], uint32_t l) {
    const bool h = l >= 4, b0 = l & 1, b1 = (l >> 1) & 1;
    rs_step<kDppHalfMirror, N>(v, h);
    rs_step<kDppXor1, (N >= 2 ? N / 2 : 1)>(v, b0);
    rs_step<kDppXor2, (N >= 4 ? N / 4 : 1)>(v, b1);
}
template <int N>
__device__ __forceinline__ uint32_t rs_item(uint32_t l) {
    const uint32_t h = l >= 4, b0 = l & 1, b1 = (l >> 1) & 1;
    return (N >= 2 ? h * (N / 2) : 0) + (N >= 4 ? b0 * (N / 4) : 0) + (N >= 8 ? b1 * (N / 8) : 0);
}
template <int N>
__device__ __forceinline__ bool rs_writer(uint32_t l) {
    const uint32_t h = l >= 4, b0 = l & 1, b1 = (l >> 1) & 1;
    return (N >= 2 || !h) && (N >= 4 || !b0) && (N >= 8 || !b1);
}

// fp32 form of reduce_scatter8 for the propagate's 32-column dots: both
// halves are summed with DPP-sourced adds (no separate lane moves) and each
// lane keeps its half, so a step costs 3 VALU per kept item.  The 4-column
// lane pieces are fp32 already; summing the 8 pieces in fp32 adds three
// roundings (relative ~2e-7 of the sum of |pieces|).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
template <int CTRL, int N>
__device__ __forceinline__ void rs_step_f32(float (&v)[8], bool upper) {
    if (N == 1) {
        v[0] += dpp_f32<CTRL>(v[0]);
        return;
    }
    constexpr int M = N / 2;
#pragma unroll
    for (int j = 0; j < M; j++) {
        const float lo = v[j] + dpp_f32<CTRL>(v[j]);
        const float hi = v[M + j] + dpp_f32<CTRL>(v[M + j]);
        v[j] = upper ? hi : lo;
    }
}
template <int N>
__device__ __forceinline__ void reduce_scatter8_f32(float (&v)[8], uint32_t l) {
    const bool h = l >= 4, b0 = l & 1, b1 = (l >> 1) & 1;
    rs_step_f32<kDppHalfMirror, N>(v, h);
    rs_step_f32<kDppXor1, (N >= 2 ? N / 2 : 1)>(v, b0);
    rs_step_f32<kDppXor2, (N >= 4 ? N / 4 : 1)>(v, b1);
}

// The lane's 4-column pieces of (W[main] - W[alt]) . g for its SPT samples of
// one staged table.  keys[] hold the two rows' byte offsets; all keys are read
// first, then the rows of 4 samples at a time, so that 8 row reads are in
// flight per wave (32 VGPRs of rows).
template <int SPT>
__device__ __forceinline__ void propagate_pieces(const uint8_t *tq, const uint32_t *keys,
                                                 uint32_t s_loc0, const f32x4 (&gv)[SPT],
                                                 float (&dv)[8]) {
    uint32_t kk[SPT];
#pragma unroll
    for (int i = 0; i < SPT; i++) kk[i] = keys[s_loc0 + kTmPass * i];
    constexpr int G = SPT < 4 ? SPT : 4;
#pragma unroll
    for (int h = 0; h < SPT; h += G) {
        f32x4 a[G], e[G];
#pragma unroll
        for (int j = 0; j < G; j++) {
            a[j] = *reinterpret_cast<const f32x4 *>(tq + (kk[h + j] & 0xFFFFu));
            e[j] = *reinterpret_cast<const f32x4 *>(tq + (kk[h + j] >> 16));
        }
#pragma unroll
        for (int j = 0; j < G; j++) {
            const f32x4 &g = gv[h + j];
            // the lane's 4-column piece in fp32 (error ~1e-7 of its terms)
            float d = (a[j].x - e[j].x) * g.x;
            d = __builtin_fmaf(a[j].y - e[j].y, g.y, d);
            d = __builtin_fmaf(a[j].z - e[j].z, g.z, d);
            d = __builtin_fmaf(a[j].w - e[j].w, g.w, d);
            dv[h + j] = d;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// LDS image of one table in a stage: E rows x 128 bytes, then one key per
// sample of the chunk (u8 row index for the forward, u16 main|alt<<8 for the
// propagate).
template <typename KEY, int SPT>
struct StageLayout {
    static constexpr int kKeys = kTmPass * SPT;
    static constexpr int kTableBytes = kTmMaxEntries * 128 + kKeys * (int)sizeof(KEY);
    static constexpr int kStageBytes = kTmPF * kTableBytes;
};

// Each thread's share of one stage: row chunks c = tid and tid + 1024 (E <= 256
// rows x 8 chunks of 16 bytes), and for the first kKeyPieces threads one
// 8-byte piece of the stage's key row (8-byte pieces keep the staging
// registers every thread carries to two per table).
template <typename KEY, int SPT>
struct KeyPieces {
    static constexpr int kPer = 8 / (int)sizeof(KEY);
    static constexpr int kCount = StageLayout<KEY, SPT>::kKeys / kPer;
};

// What a thread holds of a stage between its loads and its LDS writes: fp32
// quads, or for int8 tables the raw 4-byte words and the tables' scales,
// converted when written (4x fewer staging registers).
template <typename WT>
struct StageRaw {
    typedef f32x4 type;
};
template <>
struct StageRaw<int8_t> {
    typedef uint32_t type;
};
template <typename WT>
__device__ __forceinline__ typename StageRaw<WT>::type load_raw(const WT *p);
template <>
__device__ __forceinline__ f32x4 load_raw<float>(const float *p) {
    return *reinterpret_cast<const f32x4 *>(p);
}
template <>
__device__ __forceinline__ uint32_t load_raw<int8_t>(const int8_t *p) {
    return *reinterpret_cast<const uint32_t *>(p);
}
__device__ __forceinline__ f32x4 raw_quad(const f32x4 &v, float) { return v; }
__device__ __forceinline__ f32x4 raw_quad(uint32_t raw, float sc) {
    return f32x4{sc * (float)(int8_t)(raw & 0xFFu), sc * (float)(int8_t)((raw >> 8) & 0xFFu),
                 sc * (float)(int8_t)((raw >> 16) & 0xFFu), sc * (float)(int8_t)(raw >> 24)};
}

template <typename KEY, int SPT, typename WT = float>
__device__ __forceinline__ void stage_load(typename StageRaw<WT>::type (&rows)[kTmPF][2],
                                           float (&scs)[kTmPF], u32x2 (&keys)[kTmPF],
                                           const WT *__restrict__ w,
                                           const KEY *__restrict__ keys_t, uint32_t tid,
                                           uint32_t t_first, uint32_t nt, uint32_t n_entries,
                                           uint32_t n_outputs, uint32_t col0, uint32_t batch,
                                           uint32_t b_base, const float *__restrict__ scales = nullptr) {
    constexpr int kPer = KeyPieces<KEY, SPT>::kPer;
#pragma unroll
    for (int p = 0; p < kTmPF; p++) {
        const uint32_t t = t_first + min((uint32_t)p, nt - 1);
        const WT *wt = w + (size_t)t * n_entries * n_outputs;
        scs[p] = scales ? scales[t] : 1.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t c = tid + (uint32_t)h * kTmThreads;
            const uint32_t row = (c >> 3) & (n_entries - 1);
            uint32_t col = col0 + (c & 7) * 4;
            if (col >= n_outputs) col = 0;
            rows[p][h] = load_raw<WT>(wt + (size_t)row * n_outputs + col);
        }
        if ((int)tid < KeyPieces<KEY, SPT>::kCount) {
            // keys of samples b_base + tid*kPer .. +kPer-1 (zero past the batch)
            const uint32_t b = b_base + tid * kPer;
            const KEY *src = keys_t + (size_t)t * batch + b;
            if (b + kPer <= batch && batch % kPer == 0) {
                keys[p] = *reinterpret_cast<const u32x2 *>(src);
            } else {
                uint32_t wd[2] = {0u, 0u};
#pragma unroll
                for (int q = 0; q < kPer; q++) {
                    const uint32_t v = (b + q < batch) ? (uint32_t)src[q] : 0u;
                    wd[q / (4 / (int)sizeof(KEY))] |= v << (8 * sizeof(KEY) * (q % (4 / (int)sizeof(KEY))));
                }
                keys[p] = u32x2{wd[0], wd[1]};
            }
        }
    }
}

template <typename KEY, int SPT, typename RT>
__device__ __forceinline__ void stage_store(const RT (&rows)[kTmPF][2], const float (&scs)[kTmPF],
                                            const u32x2 (&keys)[kTmPF], uint8_t *stage,
                                            uint32_t tid) {
#pragma unroll
    for (int p = 0; p < kTmPF; p++) {
        uint8_t *tb = stage + p * StageLayout<KEY, SPT>::kTableBytes;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t c = tid + (uint32_t)h * kTmThreads;
            *reinterpret_cast<f32x4 *>(tb + c * 16) = raw_quad(rows[p][h], scs[p]);
        }
        if ((int)tid < KeyPieces<KEY, SPT>::kCount)
            *reinterpret_cast<u32x2 *>(tb + kTmMaxEntries * 128 + tid * 8) = keys[p];
    }
}

// ---------------------------------------------------------------------------
// Forward partials.  part[k][b][o] = commit value of table block k for (b, o).
// ---------------------------------------------------------------------------
// Workgroups are dealt to the 8 XCDs round robin (workgroup i runs on XCD
// i % 8).  The forward maps the n_slices column slices of one unit of tables
// to consecutive workgroups of the same XCD, so that the slices of a table row
// are fetched together, from one XCD, while they run side by side: whole 4 KiB
// rows reach HBM at once instead of 128-byte pieces spread over all XCDs
// (config 3: 2.04 -> 1.80 ms).  Grids that are not a whole number of
// 8 * n_slices workgroups keep the plain order.
__device__ __forceinline__ void xcd_slice_unit(uint32_t n_slices, uint32_t &slice, uint32_t &rest) {
    if (gridDim.x % (8u * n_slices) == 0) {
        const uint32_t local = blockIdx.x / 8u;
        slice = local % n_slices;
        rest = (local / n_slices) * 8u + blockIdx.x % 8u;
    } else {
        slice = blockIdx.x % n_slices;
        rest = blockIdx.x / n_slices;
    }
}

// A unit covers bpu consecutive blocks of dgs tables (bpu = 1 for fp32 sums;
// int32 payloads, whose wrapping sum is associative, may fold several blocks
// into one partial).  Each block's payload is formed from its own fp64 sum.
template <int SPT, bool INT_MODE, typename WT = float>
__global__ __launch_bounds__(kTmThreads) void k_fill_tm(
    const WT *__restrict__ w, const float *__restrict__ scales, const uint8_t *__restrict__ idx_t,
    uint32_t *__restrict__ part, uint32_t batch, uint32_t n_outputs, uint32_t n_detectors,
    uint32_t n_entries, uint32_t dgs, uint32_t bpu, uint32_t n_slices, uint32_t n_chunks,
    double int_rescaler) {
    using L = StageLayout<uint8_t, SPT>;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * L::kStageBytes];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = tid / kWave;
    uint32_t slice, rest;
    xcd_slice_unit(n_slices, slice, rest);
    const uint32_t chunk = rest % n_chunks;
    const uint32_t k = rest / n_chunks;
    const uint32_t t0 = k * dgs * bpu;
    const uint32_t t1 = min(t0 + dgs * bpu, n_detectors);
    const uint32_t b_base = chunk * (kTmPass * SPT);
    const uint32_t col0 = slice * kTmCols;
    const uint32_t q = lane & 7;
    const uint32_t col = col0 + q * 4;
    const uint32_t s_loc0 = wave * 8 + (lane >> 3);

    double acc[SPT][4];
    int32_t ipay[SPT][4];
#pragma unroll
    for (int i = 0; i < SPT; i++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            acc[i][c] = 0.0;
            ipay[i][c] = 0;
        }

    const uint32_t nt_all = t1 - t0;
    const uint32_t n_stages = (nt_all + kTmPF - 1) / kTmPF;
    typename StageRaw<WT>::type rows[kTmPF][2];
    float scs[kTmPF];
    u32x2 keys4[kTmPF];
    stage_load<uint8_t, SPT, WT>(rows, scs, keys4, w, idx_t, tid, t0, min((uint32_t)kTmPF, nt_all), n_entries,
                                 n_outputs, col0, batch, b_base, scales);
    for (uint32_t st = 0; st < n_stages; st++) {
        uint8_t *stage = smem + (st & 1) * L::kStageBytes;
        stage_store<uint8_t, SPT>(rows, scs, keys4, stage, tid);
        const uint32_t ts = t0 + st * kTmPF;
        const uint32_t nt = min((uint32_t)kTmPF, t1 - ts);
        if (st + 1 < n_stages) {
            const uint32_t tn = ts + kTmPF;
            stage_load<uint8_t, SPT, WT>(rows, scs, keys4, w, idx_t, tid, tn, min((uint32_t)kTmPF, t1 - tn),
                                         n_entries, n_outputs, col0, batch, b_base, scales);
        }
        __syncthreads();
        for (uint32_t p = 0; p < nt; p++) {
            const uint8_t *tb = stage + p * L::kTableBytes;
            const uint8_t *keys = tb + kTmMaxEntries * 128;
#pragma unroll
            for (int i = 0; i < SPT; i++) {
                const uint32_t r = (uint32_t)keys[s_loc0 + kTmPass * i];  // masked by k_transpose_idx
                const f32x4 v = *reinterpret_cast<const f32x4 *>(tb + r * 128 + q * 16);
                acc[i][0] += (double)v.x;
                acc[i][1] += (double)v.y;
                acc[i][2] += (double)v.z;
                acc[i][3] += (double)v.w;
            }
            // end of a block of dgs tables: its int32 payload joins the unit's sum
            const uint32_t tt = ts + p + 1;
            if (INT_MODE && ((tt - t0) % dgs == 0 || tt == t1)) {
#pragma unroll
                for (int i = 0; i < SPT; i++)
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        ipay[i][c] = wrap_add(ipay[i][c], (int32_t)(acc[i][c] * kDenom32 * int_rescaler));
                        acc[i][c] = 0.0;
                    }
            }
        }
    }
    if (col >= n_outputs) return;
#pragma unroll
    for (int i = 0; i < SPT; i++) {
        const uint32_t b = b_base + s_loc0 + kTmPass * i;
        if (b >= batch) continue;
        uint4 o;
        if (INT_MODE) {
            o.x = (uint32_t)ipay[i][0];
            o.y = (uint32_t)ipay[i][1];
            o.z = (uint32_t)ipay[i][2];
            o.w = (uint32_t)ipay[i][3];
        } else {
            o.x = __float_as_uint((float)acc[i][0]);
            o.y = __float_as_uint((float)acc[i][1]);
            o.z = __float_as_uint((float)acc[i][2]);
            o.w = __float_as_uint((float)acc[i][3]);
        }
        // written once, read once by the commit kernel: non-temporal
        __builtin_nontemporal_store(
            u32x4{o.x, o.y, o.z, o.w},
            reinterpret_cast<u32x4 *>(part + ((size_t)k * batch + b) * n_outputs + col));
    }
}

// ---------------------------------------------------------------------------
// Forward partials, LDS-DMA form (fp32 tables with 256 entries): a ring of
// kDmaRing one-table stages in LDS, filled by global_load_lds_dwordx4 three
// tables ahead (no staging registers).  Lane l of a wave writes 16 bytes at
// the wave's LDS base + 16 l, so chunk c of a stage (row c / 8, column quad
// c % 8) lands at byte 16 c: the [row][128 B] image the compute reads.  The
// stage's keys (SPT * 128 samples, u8) come from a transposed index padded to
// whole chunks of samples, loaded by wave 0.  Each wave waits for its own
// loads with an explicit vmcnt, then the workgroup barrier publishes the
// stage.  Arithmetic and partials are those of k_fill_tm.
// ---------------------------------------------------------------------------
constexpr int kDmaRing = 4;
constexpr int kDmaRows = kTmMaxEntries * 128;  // bytes of a stage's rows

typedef __attribute__((address_space(3))) void lds_void;

// AUX is the load's cache policy: 0 default, kNonTemporal for table bytes that
// are streamed once (measured 11% faster for a pure table stream on gfx950)
constexpr int kNonTemporal = 2;
template <int AUX = 0>
__device__ __forceinline__ void dma16(const void *g, void *lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *)lds_base, 16, 0, AUX);
}

// wait until at most N of this wave's vector-memory loads are outstanding
__device__ __forceinline__ void wait_vm(uint32_t n) {
    switch (n) {
        case 0: __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        case 1: __asm__ volatile("s_waitcnt vmcnt(1)" ::: "memory"); break;
        case 2: __asm__ volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
        case 3: __asm__ volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
        case 4: __asm__ volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
        case 5: __asm__ volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
        default: __asm__ volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    }
}

// RING stages, RING - 1 tables ahead.
template <int SPT, bool INT_MODE, int RING>
__global__ __launch_bounds__(kTmThreads) void k_fill_tm_dma(
    const float *__restrict__ w, const uint8_t *__restrict__ idx_t, uint32_t *__restrict__ part,
    uint32_t batch, uint32_t pitch, uint32_t n_outputs, uint32_t n_detectors, uint32_t dgs,
    uint32_t bpu, uint32_t n_slices, uint32_t n_chunks, double int_rescaler) {
    constexpr int kKeyBytes = kTmPass * SPT;
    constexpr int kStage = kDmaRows + kKeyBytes;
    __shared__ __attribute__((aligned(16))) uint8_t smem[RING * kStage];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    uint32_t slice, rest;
    xcd_slice_unit(n_slices, slice, rest);
    const uint32_t chunk = rest % n_chunks;
    const uint32_t k = rest / n_chunks;
    const uint32_t t0 = k * dgs * bpu;
    const uint32_t t1 = min(t0 + dgs * bpu, n_detectors);
    const uint32_t b_base = chunk * kKeyBytes;
    const uint32_t col0 = slice * kTmCols;
    const uint32_t q = lane & 7;
    const uint32_t col = col0 + q * 4;
    const uint32_t s_loc0 = wave * 8 + (lane >> 3);
    // this thread's two row chunks of every stage
    uint32_t goff[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t c = tid + (uint32_t)h * kTmThreads;
        uint32_t cc = col0 + (c & 7) * 4;
        if (cc >= n_outputs) cc = 0;
        goff[h] = (c >> 3) * n_outputs + cc;
    }
    const uint32_t n_loads = wave == 0 ? 3u : 2u;  // per stage, this wave
    auto issue = [&](uint32_t si) {
        const uint32_t t = t0 + si;
        uint8_t *stage = smem + (si % RING) * kStage;
        const float *wt = w + (size_t)t * kTmMaxEntries * n_outputs;
#pragma unroll
        for (int h = 0; h < 2; h++)
            dma16<kNonTemporal>(wt + goff[h], stage + ((uint32_t)h * kTmThreads + wave * kWave) * 16);
        if (wave == 0) {
            // the stage's keys: kKeyBytes bytes, 16 per lane of the first lanes
            if (lane * 16 < (uint32_t)kKeyBytes)
                dma16(idx_t + (size_t)t * pitch + b_base + lane * 16, stage + kDmaRows);
        }
    };

    double acc[SPT][4];
    int32_t ipay[SPT][4];
#pragma unroll
    for (int i = 0; i < SPT; i++)
#pragma unroll
        for (int c = 0; c < 4; c++) {
            acc[i][c] = 0.0;
            ipay[i][c] = 0;
        }
    const uint32_t nt = t1 - t0;
    for (uint32_t si = 0; si < min((uint32_t)(RING - 1), nt); si++) issue(si);
    for (uint32_t st = 0; st < nt; st++) {
        // stages issued so far: 0 .. min(st + ring - 2, nt - 1); wait for st's
        wait_vm(min((uint32_t)(RING - 2), nt - 1 - st) * n_loads);
        // stage st visible to all waves; every wave is done with stage st - 1
        // (its reads of it were consumed).  A bare s_barrier: __syncthreads'
        // fence would also wait for the later stages' loads.
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        if (st + RING - 1 < nt) issue(st + RING - 1);
        const uint8_t *tb = smem + (st % RING) * kStage;
        const uint8_t *keys = tb + kDmaRows;
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            const uint32_t r = (uint32_t)keys[s_loc0 + kTmPass * i];
            const f32x4 v = *reinterpret_cast<const f32x4 *>(tb + r * 128 + q * 16);
            acc[i][0] += (double)v.x;
            acc[i][1] += (double)v.y;
            acc[i][2] += (double)v.z;
            acc[i][3] += (double)v.w;
        }
        const uint32_t tt = t0 + st + 1;
        if (INT_MODE && ((tt - t0) % dgs == 0 || tt == t1)) {
#pragma unroll
            for (int i = 0; i < SPT; i++)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    ipay[i][c] = wrap_add(ipay[i][c], (int32_t)(acc[i][c] * kDenom32 * int_rescaler));
                    acc[i][c] = 0.0;
                }
        }
    }
    if (col >= n_outputs) return;
#pragma unroll
    for (int i = 0; i < SPT; i++) {
        const uint32_t b = b_base + s_loc0 + kTmPass * i;
        if (b >= batch) continue;
        uint4 o;
        if (INT_MODE) {
            o = make_uint4((uint32_t)ipay[i][0], (uint32_t)ipay[i][1], (uint32_t)ipay[i][2],
                           (uint32_t)ipay[i][3]);
        } else {
            o = make_uint4(__float_as_uint((float)acc[i][0]), __float_as_uint((float)acc[i][1]),
                           __float_as_uint((float)acc[i][2]), __float_as_uint((float)acc[i][3]));
        }
        __builtin_nontemporal_store(
            u32x4{o.x, o.y, o.z, o.w},
            reinterpret_cast<u32x4 *>(part + ((size_t)k * batch + b) * n_outputs + col));
    }
}

// out[b][o] (+)= sum over blocks k ascending of part[k][b][o] (fp32 or int32).
template <bool INT_MODE>
__global__ __launch_bounds__(256) void k_fill_commit(const uint32_t *__restrict__ part,
                                                     float *__restrict__ out, uint64_t n_quads,
                                                     uint32_t n_blocks, uint64_t stride,
                                                     double int_rescaler) {
    const uint64_t qd = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (qd >= n_quads) return;
    float4 *op = reinterpret_cast<float4 *>(out) + qd;
    const uint4 *pp = reinterpret_cast<const uint4 *>(part) + qd;
    const uint64_t s4 = stride / 4;
    float4 run = *op;
    int32_t ir[4] = {__float_as_int(run.x), __float_as_int(run.y), __float_as_int(run.z),
                     __float_as_int(run.w)};
    uint32_t k = 0;
    constexpr int kU = 16;  // loads in flight a thread (config 3: 0.219 ms; 0.225 ms with 8)
    for (; k + kU <= n_blocks; k += kU) {
        uint4 v[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) v[u] = pp[(k + u) * s4];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            if (INT_MODE) {
                ir[0] = wrap_add(ir[0], (int32_t)v[u].x);
                ir[1] = wrap_add(ir[1], (int32_t)v[u].y);
                ir[2] = wrap_add(ir[2], (int32_t)v[u].z);
                ir[3] = wrap_add(ir[3], (int32_t)v[u].w);
            } else {
                run.x += __uint_as_float(v[u].x);
                run.y += __uint_as_float(v[u].y);
                run.z += __uint_as_float(v[u].z);
                run.w += __uint_as_float(v[u].w);
            }
        }
    }
    for (; k < n_blocks; k++) {
        const uint4 v = pp[k * s4];
        if (INT_MODE) {
            ir[0] = wrap_add(ir[0], (int32_t)v.x);
            ir[1] = wrap_add(ir[1], (int32_t)v.y);
            ir[2] = wrap_add(ir[2], (int32_t)v.z);
            ir[3] = wrap_add(ir[3], (int32_t)v.w);
        } else {
            run.x += __uint_as_float(v.x);
            run.y += __uint_as_float(v.y);
            run.z += __uint_as_float(v.z);
            run.w += __uint_as_float(v.w);
        }
    }
    if (INT_MODE) {
        // convert_integers_to_floats_logic, proto:200-213
        run.x = (float)(((double)ir[0] * kDenom32Reciproc) / int_rescaler);
        run.y = (float)(((double)ir[1] * kDenom32Reciproc) / int_rescaler);
        run.z = (float)(((double)ir[2] * kDenom32Reciproc) / int_rescaler);
        run.w = (float)(((double)ir[3] * kDenom32Reciproc) / int_rescaler);
    }
    *op = run;
}

// ---------------------------------------------------------------------------
// Propagate partials.  dpart[s][t][b] = fp32(sum over slice s's columns of
// (W[t][main] - W[t][alt]) * g[b]).  Key = main * 128 | (alt * 128) << 16: the
// two rows' byte offsets in the stage.
// ---------------------------------------------------------------------------
template <int SPT>
__global__ __launch_bounds__(kTmThreads) void k_propagate_tm(
    const float *__restrict__ w, const float *__restrict__ g, const uint32_t *__restrict__ key_t,
    float *__restrict__ dpart, uint32_t batch, uint32_t pitch, uint32_t n_outputs,
    uint32_t n_detectors, uint32_t n_entries, uint32_t tpu, uint32_t n_slices, uint32_t n_chunks) {
    using L = StageLayout<uint32_t, SPT>;
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * L::kStageBytes];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = tid / kWave;
    const uint32_t slice = blockIdx.x % n_slices;
    const uint32_t rest = blockIdx.x / n_slices;
    const uint32_t chunk = rest % n_chunks;
    const uint32_t k = rest / n_chunks;
    const uint32_t t0 = k * tpu;
    const uint32_t t1 = min(t0 + tpu, n_detectors);
    const uint32_t b_base = chunk * (kTmPass * SPT);
    const uint32_t col0 = slice * kTmCols;
    const uint32_t q = lane & 7;
    const uint32_t col = col0 + q * 4;
    const bool active = col < n_outputs;
    const uint32_t s_loc0 = wave * 8 + (lane >> 3);

    f32x4 gv[SPT];
#pragma unroll
    for (int i = 0; i < SPT; i++) {
        const uint32_t b = min(b_base + s_loc0 + kTmPass * i, batch - 1);
        gv[i] = active ? *reinterpret_cast<const f32x4 *>(g + (size_t)b * n_outputs + col)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
    }

    const uint32_t nt_all = t1 - t0;
    const uint32_t n_stages = (nt_all + kTmPF - 1) / kTmPF;
    f32x4 rows[kTmPF][2];
    float scs[kTmPF];
    u32x2 keys4[kTmPF];
    // keys rows have `pitch` (a whole number of chunks, zero past the batch)
    stage_load<uint32_t, SPT>(rows, scs, keys4, w, key_t, tid, t0, min((uint32_t)kTmPF, nt_all), n_entries,
                              n_outputs, col0, pitch, b_base);
    for (uint32_t st = 0; st < n_stages; st++) {
        uint8_t *stage = smem + (st & 1) * L::kStageBytes;
        stage_store<uint32_t, SPT>(rows, scs, keys4, stage, tid);
        const uint32_t ts = t0 + st * kTmPF;
        const uint32_t nt = min((uint32_t)kTmPF, t1 - ts);
        if (st + 1 < n_stages) {
            const uint32_t tn = ts + kTmPF;
            stage_load<uint32_t, SPT>(rows, scs, keys4, w, key_t, tid, tn, min((uint32_t)kTmPF, t1 - tn),
                                      n_entries, n_outputs, col0, pitch, b_base);
        }
        __syncthreads();
        for (uint32_t p = 0; p < nt; p++) {
            const uint8_t *tb = stage + p * L::kTableBytes;
            const uint32_t *keys = reinterpret_cast<const uint32_t *>(tb + kTmMaxEntries * 128);
            const uint8_t *tq = tb + q * 16;
            const uint32_t t = ts + p;
            float dv[8];
            propagate_pieces<SPT>(tq, keys, s_loc0, gv, dv);
            // the 8 lanes of a sample group each hold a 4-column piece of the
            // SPT dots; after the reduce-scatter lane q holds sample rs_item's sum
            reduce_scatter8_f32<SPT>(dv, q);
            const uint32_t b = b_base + s_loc0 + kTmPass * rs_item<SPT>(q);
            if (rs_writer<SPT>(q) && b < batch)
                // 4-byte pieces of 4 KiB table rows: plain stores, so that L2
                // merges them into full lines before they reach HBM
                dpart[((size_t)slice * n_detectors + t) * batch + b] = dv[0];
        }
    }
}

// Propagate partials, LDS-DMA form (fp32 tables with 256 entries): the ring of
// k_fill_tm_dma, with the stage's u32 keys (the two rows' byte offsets) loaded by the
// first kKeyWaves waves from keys transposed to a row pitch that is a whole
// number of sample chunks.  Arithmetic and partials are those of
// k_propagate_tm.
template <int SPT, int RING>
__global__ __launch_bounds__(kTmThreads) void k_propagate_tm_dma(
    const float *__restrict__ w, const float *__restrict__ g, const uint32_t *__restrict__ key_t,
    float *__restrict__ dpart, uint32_t batch, uint32_t pitch, uint32_t n_outputs,
    uint32_t n_detectors, uint32_t tpu, uint32_t n_slices, uint32_t n_chunks) {
    constexpr int kKeyBytes = kTmPass * SPT * 4;
    constexpr int kStage = kDmaRows + kKeyBytes;
    constexpr uint32_t kKeyWaves = (kKeyBytes + kWave * 16 - 1) / (kWave * 16);
    __shared__ __attribute__((aligned(16))) uint8_t smem[RING * kStage];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    // wave-uniform: the per-wave load count and vmcnt wait stay scalar
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t slice = blockIdx.x % n_slices;
    const uint32_t rest = blockIdx.x / n_slices;
    const uint32_t chunk = rest % n_chunks;
    const uint32_t k = rest / n_chunks;
    const uint32_t t0 = k * tpu;
    const uint32_t t1 = min(t0 + tpu, n_detectors);
    const uint32_t b_base = chunk * (kTmPass * SPT);
    const uint32_t col0 = slice * kTmCols;
    const uint32_t q = lane & 7;
    const uint32_t col = col0 + q * 4;
    const bool active = col < n_outputs;
    const uint32_t s_loc0 = wave * 8 + (lane >> 3);

    f32x4 gv[SPT];
#pragma unroll
    for (int i = 0; i < SPT; i++) {
        const uint32_t b = min(b_base + s_loc0 + kTmPass * i, batch - 1);
        gv[i] = active ? *reinterpret_cast<const f32x4 *>(g + (size_t)b * n_outputs + col)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    uint32_t goff[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t c = tid + (uint32_t)h * kTmThreads;
        uint32_t cc = col0 + (c & 7) * 4;
        if (cc >= n_outputs) cc = 0;
        goff[h] = (c >> 3) * n_outputs + cc;
    }
    const uint32_t n_loads = wave < kKeyWaves ? 3u : 2u;  // per stage, this wave
    auto issue = [&](uint32_t si) {
        const uint32_t t = t0 + si;
        uint8_t *stage = smem + (si % RING) * kStage;
        const float *wt = w + (size_t)t * kTmMaxEntries * n_outputs;
#pragma unroll
        for (int h = 0; h < 2; h++)
            dma16(wt + goff[h], stage + ((uint32_t)h * kTmThreads + wave * kWave) * 16);
        if (wave < kKeyWaves) {
            const uint32_t byte = wave * kWave * 16 + lane * 16;
            if (byte < (uint32_t)kKeyBytes)
                dma16(reinterpret_cast<const uint8_t *>(key_t + (size_t)t * pitch + b_base) + byte,
                      stage + kDmaRows + wave * kWave * 16);
        }
    };

    const uint32_t nt = t1 - t0;
    for (uint32_t si = 0; si < min((uint32_t)(RING - 1), nt); si++) issue(si);
    for (uint32_t st = 0; st < nt; st++) {
        wait_vm(min((uint32_t)(RING - 2), nt - 1 - st) * n_loads);
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        if (st + RING - 1 < nt) issue(st + RING - 1);
        const uint8_t *tb = smem + (st % RING) * kStage;
        const uint32_t *keys = reinterpret_cast<const uint32_t *>(tb + kDmaRows);
        const uint8_t *tq = tb + q * 16;
        const uint32_t t = t0 + st;
        float dv[8];
        propagate_pieces<SPT>(tq, keys, s_loc0, gv, dv);
        reduce_scatter8_f32<SPT>(dv, q);
        const uint32_t b = b_base + s_loc0 + kTmPass * rs_item<SPT>(q);
        if (rs_writer<SPT>(q) && b < batch)
            dpart[((size_t)slice * n_detectors + t) * batch + b] = dv[0];
    }
}

// Propagate over whole tables (fp32 tables with 256 entries, n_outputs % 64 ==
// 0).  A unit is TPU tables x every 64-column slice x one chunk of SPT * 128
// samples.  The slice loop is outside the table loop: the slice's g columns
// sit in registers (64 VGPRs at SPT = 8) while its TPU table stages stream
// through a two-stage LDS-DMA ring (256 rows x 256 bytes each, the rows'
// 256-byte HBM pieces loaded non-temporally), and every lane keeps one fp32
// accumulator per table for one sample: the reference's per-(table, 32-output
// block) terms du * (main - alt) of all the slices (proto:1421-1499, each
// dropped unless |term| > EPS, proto:833-863).  du[b][t] is written once per
// unit, so no per-slice partial crosses HBM (gfx950 pays about ten times a
// read for a write mixed into a saturated read stream: config 3's 537 MB of
// per-slice partials cost about 0.4 ms).
//
// Thread layout: wave w, lane l; sample group grp = l / 8 of the wave owns
// sample w * 8 + grp (+128 i, i < SPT) and lane q = l % 8 the columns 8q ..
// 8q + 7 of the slice, read as two 16-byte LDS pieces in swapped order on odd
// groups (the two groups of a 16-lane LDS service group then read disjoint
// bank halves of their rows).  Keys are the rows' byte offsets in a stage,
// main * 256 | (alt * 256) << 16, and du_t[t][b] is du(min margin) (0 when
// the sample's min-margin index is unused), both with the key pitch.
constexpr int kUnitPass = (kTmThreads / kWave) * 8;  // samples per pass: 128
constexpr int kTm64Rows = kTmMaxEntries * 256;       // bytes of a stage's rows

template <int SPT, int TPU>
__global__ __launch_bounds__(kTmThreads) void k_propagate_units(
    const float *__restrict__ w, const float *__restrict__ g, const uint32_t *__restrict__ key_t,
    const float *__restrict__ du_t, float *__restrict__ du_out, uint32_t batch, uint32_t pitch,
    uint32_t n_outputs, uint32_t n_detectors, uint32_t n_chunks, bool block_eps) {
    static_assert(SPT == 4 || SPT == 8, "one or two groups of four samples a lane");
    constexpr int kKeyBytes = kUnitPass * SPT * 4;    // keys, then as many bytes of du
    constexpr int kStage = kTm64Rows + 2 * kKeyBytes;
    constexpr uint32_t kKeyWaves = (kKeyBytes + kWave * 16 - 1) / (kWave * 16);
    constexpr int kRowLoads = kTm64Rows / (kTmThreads * 16);
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kStage];
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & (kWave - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const uint32_t chunk = blockIdx.x % n_chunks;
    const uint32_t t0 = (blockIdx.x / n_chunks) * TPU;
    const uint32_t ntab = min((uint32_t)TPU, n_detectors - t0);
    const uint32_t n_slices = n_outputs / 64;
    const uint32_t b_base = chunk * (kUnitPass * SPT);
    const uint32_t q = lane & 7;
    const uint32_t grp = lane >> 3;
    const uint32_t sw = (grp & 1) * 16;
    const uint32_t s_loc0 = wave * 8 + grp;
    // lanes q < 4 sum the slice's first 32-column block, lanes q >= 4 its
    // second; lane q and lane 7 - q hold the same samples after each quad
    // reduction, so one half-mirror exchange joins a sample's two blocks
    const bool hi = q >= 4;
    const uint32_t qm = hi ? 7 - q : q;
    const bool c1 = (qm >> 1) & 1, c0 = qm & 1;
    const uint32_t my_item = (hi && SPT == 8 ? 4u : 0u) + 2 * c1 + c0;
    const bool writer = SPT == 8 || !hi;
    const uint32_t my_b = b_base + s_loc0 + kUnitPass * my_item;

    float acc[TPU];
#pragma unroll
    for (int j = 0; j < TPU; j++) acc[j] = 0.0f;
    f32x4 g0[SPT], g1[SPT];
    // g by buffer loads with 32-bit byte offsets: the lane's two 16-byte pieces
    // in VGPRs, the sample pass and the slice in the scalar offset (64-bit
    // addresses per sample pass would not fit beside g without spilling).
    // Samples past the batch lie beyond the resource and read as zeros; the
    // launcher keeps every offset below 2^31.
    const __amdgpu_buffer_rsrc_t g_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)g, (short)0, (int)(batch * n_outputs * 4u), 0x00020000);
    const uint32_t g_lane = ((b_base + s_loc0) * n_outputs + q * 8) * 4u;
    const uint32_t g_v0 = g_lane + sw, g_v1 = g_lane + 16 - sw;
    const uint32_t n_st = ntab * n_slices;
    auto issue = [&](uint32_t si) {
        const uint32_t sl = si / ntab, t = t0 + si % ntab;
        uint8_t *stage = smem + (si & 1) * kStage;
        const float *wt = w + (size_t)t * kTmMaxEntries * n_outputs + sl * 64;
        // keys and du first: should their address come back from a register
        // spill, the wait for that reload then finds no row load in flight
        if (wave < 2 * kKeyWaves) {
            // waves 0 .. kKeyWaves-1 load the keys, the next kKeyWaves the du values
            const bool is_du = wave >= kKeyWaves;
            const uint32_t wk = is_du ? wave - kKeyWaves : wave;
            const uint32_t byte = wk * kWave * 16 + lane * 16;
            const uint8_t *src = is_du ? reinterpret_cast<const uint8_t *>(du_t + (size_t)t * pitch + b_base)
                                       : reinterpret_cast<const uint8_t *>(key_t + (size_t)t * pitch + b_base);
            if (byte < (uint32_t)kKeyBytes)
                dma16(src + byte, stage + kTm64Rows + (is_du ? kKeyBytes : 0) + wk * kWave * 16);
        }
#pragma unroll
        for (int h = 0; h < kRowLoads; h++) {
            const uint32_t c = (uint32_t)h * kTmThreads + tid;  // row c / 16, quad c % 16
            dma16<kNonTemporal>(wt + (c >> 4) * n_outputs + (c & 15) * 4,
                                stage + ((uint32_t)h * kTmThreads + wave * kWave) * 16);
        }
    };

    issue(0);
    for (uint32_t si = 0; si < n_st; si++) {
        const uint32_t sl = si / ntab, tl = si % ntab;
        if (tl == 0) {
            // this slice's g columns, in the lane's read order
#pragma unroll
            for (int i = 0; i < SPT; i++) {
                const uint32_t so = (kUnitPass * (uint32_t)i * n_outputs + sl * 64) * 4u;
                g0[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, g_v0, so, 0));
                g1[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, g_v1, so, 0));
            }
        }
        // stage si (and the g columns) have landed; every wave is done with
        // stage si - 1, whose slot takes stage si + 1
        wait_vm(0);
        __syncthreads();
        if (si + 1 < n_st) issue(si + 1);
        const uint8_t *tb = smem + (si & 1) * kStage;
        const uint32_t *keys = reinterpret_cast<const uint32_t *>(tb + kTm64Rows);
        const float *dus = reinterpret_cast<const float *>(tb + kTm64Rows + kKeyBytes);
        const uint8_t *tq = tb + q * 32 + sw;
        float tot[SPT / 4];
#pragma unroll
        for (int h = 0; h < SPT / 4; h++) {
            // four samples at a time: the lane's 8-column pieces in fp32
            float pc[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ii = 4 * h + i;
                const uint32_t kk = keys[s_loc0 + kUnitPass * ii];
                const uint8_t *pm = tq + (kk & 0xFFFFu);
                const uint8_t *pa = tq + (kk >> 16);
                const f32x4 a0 = *reinterpret_cast<const f32x4 *>(pm);
                const f32x4 a1 = *reinterpret_cast<const f32x4 *>(pm + 16 - 2 * sw);
                const f32x4 e0 = *reinterpret_cast<const f32x4 *>(pa);
                const f32x4 e1 = *reinterpret_cast<const f32x4 *>(pa + 16 - 2 * sw);
                float d = (a0.x - e0.x) * g0[ii].x;
                d = __builtin_fmaf(a0.y - e0.y, g0[ii].y, d);
                d = __builtin_fmaf(a0.z - e0.z, g0[ii].z, d);
                d = __builtin_fmaf(a0.w - e0.w, g0[ii].w, d);
                d = __builtin_fmaf(a1.x - e1.x, g1[ii].x, d);
                d = __builtin_fmaf(a1.y - e1.y, g1[ii].y, d);
                d = __builtin_fmaf(a1.z - e1.z, g1[ii].z, d);
                d = __builtin_fmaf(a1.w - e1.w, g1[ii].w, d);
                pc[i] = d;
                // at most two samples' rows in flight (32 VGPRs): the 64 VGPRs
                // of g leave no room for more without spilling
                if (i & 1) __builtin_amdgcn_sched_barrier(0);
            }
            // quad reduce-scatter (lanes q, q ^ 2, then q, q ^ 1): lane q is
            // left with the 32-column block sum of sample 4h + 2 c1 + c0
            float r2[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float lo = pc[j] + dpp_f32<kDppXor2>(pc[j]);
                const float up = pc[2 + j] + dpp_f32<kDppXor2>(pc[2 + j]);
                r2[j] = c1 ? up : lo;
            }
            const float lo = r2[0] + dpp_f32<kDppXor1>(r2[0]);
            const float up = r2[1] + dpp_f32<kDppXor1>(r2[1]);
            const float r1 = c0 ? up : lo;
            // the reference's block term du * (main - alt), dropped unless
            // |term| > EPS (proto:833-863), then the sample's two blocks joined
            float term = dus[s_loc0 + kUnitPass * (4 * h + 2 * c1 + c0)] * r1;
            if (block_eps && !(fabsf(term) > (float)kEps)) term = 0.0f;
            tot[h] = term + dpp_f32<kDppHalfMirror>(term);
        }
        const float add = (SPT == 8 && hi) ? tot[SPT / 4 - 1] : tot[0];
#pragma unroll
        for (int j = 0; j < TPU; j++)
            if (j == (int)tl) acc[j] += add;
    }
    if (writer && my_b < batch) {
        float *dst = du_out + (size_t)my_b * n_detectors + t0;
#pragma unroll
        for (int j = 0; j < TPU; j++)
            if (j < (int)ntab) dst[j] = fabs((double)acc[j]) > kEps ? acc[j] : 0.0f;
    }
}

// du[b][t] = sum over slices s ascending of du(min margin of (b, t)) *
// dpart[s][t][b] (fp64), or 0 when the min-margin index is unused.  One
// workgroup per 64 tables x 64 samples tile; md / mi and du pass through LDS so
// that every global access is coalesced.
__global__ __launch_bounds__(256) void k_propagate_reduce(const float *__restrict__ dpart,
                                                          const float *__restrict__ md,
                                                          const int32_t *__restrict__ mi,
                                                          float *__restrict__ du_out,
                                                          uint32_t batch, uint32_t n_detectors,
                                                          uint32_t n_anchors, uint32_t n_slices,
                                                          bool per_slice_eps) {
    __shared__ float s_md[64][65];
    __shared__ int32_t s_mi[64][65];
    __shared__ float s_du[64][65];
    const uint32_t tb = blockIdx.x * 64;
    const uint32_t bb = blockIdx.y * 64;
    const uint32_t tx = threadIdx.x & 63;
    const uint32_t ty = threadIdx.x >> 6;
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t b = bb + r, t = tb + tx;
        if (b < batch && t < n_detectors) {
            s_md[r][tx] = md[(size_t)b * n_detectors + t];
            s_mi[r][tx] = mi[(size_t)b * n_detectors + t];
        }
    }
    __syncthreads();
    // thread (tx = sample, r = table): coalesced over samples
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t t = tb + r, b = bb + tx;
        float du = 0.0f;
        if (b < batch && t < n_detectors) {
            const int32_t m = s_mi[tx][r];
            if (m >= 0 && (uint32_t)m < n_anchors) {
                // slice terms du(margin) * dot; with per_slice_eps (slices are the
                // reference's 32-output blocks) each term is dropped unless
                // |term| > EPS, as the reference's per-block commit does
                // (proto:833-863, misc.h:90)
                const double dm = du_of_margin(s_md[tx][r]);
                double acc = 0.0;
                const float *p = dpart + (size_t)t * batch + b;
                const size_t stride = (size_t)n_detectors * batch;
                uint32_t s = 0;
                for (; s + 8 <= n_slices; s += 8) {
                    float v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) v[u] = p[(s + u) * stride];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        const double term = dm * (double)v[u];
                        if (!per_slice_eps || fabs(term) > kEps) acc += term;
                    }
                }
                for (; s < n_slices; s++) {
                    const double term = dm * (double)p[s * stride];
                    if (!per_slice_eps || fabs(term) > kEps) acc += term;
                }
                if (fabs(acc) > kEps) du = (float)acc;
            }
        }
        s_du[tx][r] = du;
    }
    __syncthreads();
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t b = bb + r, t = tb + tx;
        if (b < batch && t < n_detectors) du_out[(size_t)b * n_detectors + t] = s_du[r][tx];
    }
}

// x_grad[b][a1] += du, x_grad[b][a2] -= du for every table with |du| > EPS
// (propagate_through_detector, proto:821-867).  One workgroup per group of
// samples; their input-gradient rows are accumulated in LDS and added to HBM
// once.
constexpr int kScatterThreads = 1024;
constexpr int kScatterLds = 128 * 1024;

__global__ __launch_bounds__(kScatterThreads) void k_propagate_scatter(
    const float *__restrict__ du_in, const int32_t *__restrict__ mi,
    const int2 *__restrict__ anchors, float *__restrict__ x_grad, uint32_t batch,
    uint32_t n_inputs, uint32_t n_detectors, uint32_t n_anchors, uint32_t samples_per_group) {
    // fp64 sums: on gfx950 ds_add_f64 sustains ~20x the lanes a clock of ds_add_f32
    __shared__ double xg[kScatterLds / 8];
    const uint32_t b0 = blockIdx.x * samples_per_group;
    const uint32_t nb = min(samples_per_group, batch - b0);
    const uint32_t n_el = nb * n_inputs;
    for (uint32_t i = threadIdx.x; i < n_el; i += kScatterThreads) xg[i] = 0.0;
    __syncthreads();
    const uint32_t n_pairs = nb * n_detectors;
    const size_t base = (size_t)b0 * n_detectors;
    // eight (sample, table) items a thread at a time: their du and margin index
    // loads, then their anchor loads, each batch in flight together
    constexpr int kU = 8;
    for (uint32_t p0 = threadIdx.x; p0 < n_pairs; p0 += kU * kScatterThreads) {
        float du[kU];
        int32_t m[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const uint32_t p = p0 + u * kScatterThreads;
            du[u] = p < n_pairs ? du_in[base + p] : 0.0f;
            m[u] = p < n_pairs ? mi[base + p] : -1;
        }
        int2 a[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            const uint32_t t = (p0 + u * kScatterThreads) % n_detectors;
            const bool on = du[u] != 0.0f && m[u] >= 0 && (uint32_t)m[u] < n_anchors;
            a[u] = on ? anchors[(size_t)t * n_anchors + m[u]] : make_int2(-1, -1);
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            if ((uint32_t)a[u].x >= n_inputs || (uint32_t)a[u].y >= n_inputs) continue;
            const uint32_t bl = (p0 + u * kScatterThreads) / n_detectors;
            atomicAdd(&xg[bl * n_inputs + a[u].x], (double)du[u]);
            atomicAdd(&xg[bl * n_inputs + a[u].y], -(double)du[u]);
        }
    }
    __syncthreads();
    float *dst = x_grad + (size_t)b0 * n_inputs;
    for (uint32_t i = threadIdx.x; i < n_el; i += kScatterThreads) dst[i] += (float)xg[i];
}

// keys_t[t][b] = idx[b][t] & emask (u8), through a 64x64 LDS tile: the rows the
// forward reads, masked here once instead of once per column slice.
// idx_t[t][b] (row pitch `pitch` >= batch; samples past the batch get 0).
__global__ __launch_bounds__(256) void k_transpose_idx(const int32_t *__restrict__ idx,
                                                       uint8_t *__restrict__ idx_t,
                                                       uint32_t batch, uint32_t n_detectors,
                                                       uint32_t pitch, uint32_t emask) {
    __shared__ uint8_t tile[64][65];
    const uint32_t tb = blockIdx.x * 64;  // table tile
    const uint32_t bb = blockIdx.y * 64;  // sample tile
    const uint32_t tx = threadIdx.x & 63;
    const uint32_t ty = threadIdx.x >> 6;
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t b = bb + r, t = tb + tx;
        tile[r][tx] = (b < batch && t < n_detectors) ? (uint8_t)((uint32_t)idx[(size_t)b * n_detectors + t] & emask) : 0;
    }
    __syncthreads();
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t t = tb + r, b = bb + tx;
        if (b < pitch && t < n_detectors) idx_t[(size_t)t * pitch + b] = tile[tx][r];
    }
}

// keys_t[t][b] = main << row_shift | (alt << row_shift) << 16 (the rows' byte
// offsets in a stage of 128- or 256-byte rows) with alt = main ^ (1 << min_idx) (main when the
// min-margin index is unused), through a 64x64 LDS tile; row pitch `pitch` >=
// batch, samples past the batch get 0.  With du_t, also du_t[t][b] = fp32 of
// du(min margin), 0 when the min-margin index is unused.
__global__ __launch_bounds__(256) void k_transpose_keys(const int32_t *__restrict__ idx,
                                                        const int32_t *__restrict__ mi,
                                                        const float *__restrict__ md,
                                                        uint32_t *__restrict__ key_t,
                                                        float *__restrict__ du_t,
                                                        uint32_t batch, uint32_t pitch,
                                                        uint32_t n_detectors, uint32_t n_anchors,
                                                        uint32_t n_entries, uint32_t row_shift) {
    __shared__ uint32_t tile[64][65];
    __shared__ float dtile[64][65];
    const uint32_t tb = blockIdx.x * 64;
    const uint32_t bb = blockIdx.y * 64;
    const uint32_t tx = threadIdx.x & 63;
    const uint32_t ty = threadIdx.x >> 6;
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t b = bb + r, t = tb + tx;
        if (b < batch && t < n_detectors) {
            const size_t bt = (size_t)b * n_detectors + t;
            const uint32_t rm = (uint32_t)idx[bt] & (n_entries - 1);
            const int32_t m = mi[bt];
            const uint32_t ra = (m >= 0 && (uint32_t)m < n_anchors) ? (rm ^ (1u << m)) : rm;
            tile[r][tx] = (rm << row_shift) | (ra << (row_shift + 16));
            if (du_t) dtile[r][tx] = (m >= 0 && (uint32_t)m < n_anchors) ? (float)du_of_margin(md[bt]) : 0.0f;
        } else {
            tile[r][tx] = 0;
            dtile[r][tx] = 0.0f;
        }
    }
    __syncthreads();
    for (uint32_t r = ty; r < 64; r += 4) {
        const uint32_t t = tb + r, b = bb + tx;
        if (b < pitch && t < n_detectors) {
            key_t[(size_t)t * pitch + b] = tile[tx][r];
            if (du_t) du_t[(size_t)t * pitch + b] = dtile[tx][r];
        }
    }
}

// The same transpose with 16-byte accesses both ways (n_detectors % 4 == 0,
// pitch % 4 == 0): a thread reads four tables of a sample row and writes four
// samples of a table row.
__global__ __launch_bounds__(256) void k_transpose_keys4(const int32_t *__restrict__ idx,
                                                         const int32_t *__restrict__ mi,
                                                         const float *__restrict__ md,
                                                         uint32_t *__restrict__ key_t,
                                                         float *__restrict__ du_t,
                                                         uint32_t batch, uint32_t pitch,
                                                         uint32_t n_detectors, uint32_t n_anchors,
                                                         uint32_t n_entries, uint32_t row_shift) {
    __shared__ uint32_t tile[64][65];
    __shared__ float dtile[64][65];
    const uint32_t tb = blockIdx.x * 64;
    const uint32_t bb = blockIdx.y * 64;
    const uint32_t c4 = (threadIdx.x & 15) * 4;
    const uint32_t r0 = threadIdx.x >> 4;
#pragma unroll
    for (uint32_t r = r0; r < 64; r += 16) {
        const uint32_t b = bb + r, t = tb + c4;
        uint32_t k[4] = {0u, 0u, 0u, 0u};
        float dv[4] = {0.f, 0.f, 0.f, 0.f};
        if (b < batch && t < n_detectors) {
            const size_t bt = (size_t)b * n_detectors + t;
            const int4 iv = *reinterpret_cast<const int4 *>(idx + bt);
            const int4 mv = *reinterpret_cast<const int4 *>(mi + bt);
            const int ia[4] = {iv.x, iv.y, iv.z, iv.w}, ma[4] = {mv.x, mv.y, mv.z, mv.w};
            float da[4] = {0.f, 0.f, 0.f, 0.f};
            if (du_t) {
                const float4 dd = *reinterpret_cast<const float4 *>(md + bt);
                da[0] = dd.x; da[1] = dd.y; da[2] = dd.z; da[3] = dd.w;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t rm = (uint32_t)ia[c] & (n_entries - 1);
                const int32_t m = ma[c];
                const bool used = m >= 0 && (uint32_t)m < n_anchors;
                const uint32_t ra = used ? (rm ^ (1u << m)) : rm;
                k[c] = (rm << row_shift) | (ra << (row_shift + 16));
                if (du_t) dv[c] = used ? (float)du_of_margin(da[c]) : 0.0f;
            }
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            tile[r][c4 + c] = k[c];
            dtile[r][c4 + c] = dv[c];
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t r = r0; r < 64; r += 16) {
        const uint32_t t = tb + r, b = bb + c4;
        if (b < pitch && t < n_detectors) {
            *reinterpret_cast<uint4 *>(key_t + (size_t)t * pitch + b) =
                make_uint4(tile[c4][r], tile[c4 + 1][r], tile[c4 + 2][r], tile[c4 + 3][r]);
            if (du_t)
                *reinterpret_cast<float4 *>(du_t + (size_t)t * pitch + b) =
                    make_float4(dtile[c4][r], dtile[c4 + 1][r], dtile[c4 + 2][r], dtile[c4 + 3][r]);
        }
    }
}

constexpr uint64_t kFoldUnits = 1024;

uint32_t tm_spt(uint32_t batch) {
    if (batch <= (uint32_t)kTmPass) return 1;
    if (batch <= 2u * kTmPass) return 2;
    if (batch <= 4u * kTmPass) return 4;
    return 8;
}

}  // namespace

// Blocks of dgs tables per unit.  Ordered fp32 sums: 1 (every block is a
// rounding point committed in order).  int32 payloads (whose wrapping sum is
// associative): enough to leave about 2048 units.  Folded fp32 sums: enough to
// leave about 1024 units, each partial the fp64 sum of its blocks' tables --
// the partials are written while the table stream is running, and on gfx950
// a write mixed into a saturated read stream costs about ten times a read
// (config 3: 1.07 GB of per-block partials, 134 MB folded eight blocks a unit).
static uint32_t tm_fill_bpu(const FcShape &s, bool int_mode) {
    if (!int_mode && s.ordered_sums) return 1;
    const uint64_t n_blocks = (s.n_detectors + s.dgs - 1) / s.dgs;
    const uint64_t spt = tm_spt(s.batch);
    const uint64_t n_chunks = (s.batch + kTmPass * spt - 1) / (kTmPass * spt);
    const uint64_t n_slices = (s.n_outputs + kTmCols - 1) / kTmCols;
    const uint64_t units = n_blocks * n_chunks * n_slices;
    const uint64_t target = int_mode ? 2048 : kFoldUnits;
    return (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(n_blocks, units / target));
}

bool tm_fill_applies(const FcShape &s, bool int_mode) {
    const uint64_t n_blocks = (s.n_detectors + s.dgs - 1) / s.dgs;
    const uint64_t bpu = tm_fill_bpu(s, int_mode);
    return s.batch >= 256 && s.n_entries <= (uint32_t)kTmMaxEntries && s.n_outputs % 4 == 0 &&
           s.n_outputs >= 64 && s.dgs >= 8 &&
           ((n_blocks + bpu - 1) / bpu) * s.batch * s.n_outputs * 4 <= (4ull << 30);
}

// Row pitch of the transposed index: whole chunks of samples, so that every
// stage's key row can be loaded in 16-byte pieces.
static uint32_t tm_fill_pitch(const FcShape &s) {
    const uint32_t spt = tm_spt(s.batch);
    const uint32_t n_chunks = (s.batch + kTmPass * spt - 1) / (kTmPass * spt);
    return n_chunks * kTmPass * spt;
}

// scratch: u8 lookup indices transposed [T][pitch] | partials [n_parts][B][O]
// (fp32 commits, or wrapping int32 sums)
template <typename WT>
static hipError_t launch_fill_tm_impl(const FcShape &s, const WT *w, const float *scales,
                                      const int32_t *idx, float *out, bool int_mode,
                                      double int_rescaler, Scratch &scratch, hipStream_t st) {
    const uint32_t pitch = tm_fill_pitch(s);
    const uint32_t spt = tm_spt(s.batch);
    const uint32_t n_chunks = (s.batch + kTmPass * spt - 1) / (kTmPass * spt);
    const uint32_t n_slices = (s.n_outputs + kTmCols - 1) / kTmCols;
    const uint32_t n_blocks = (s.n_detectors + s.dgs - 1) / s.dgs;
    const uint32_t bpu = tm_fill_bpu(s, int_mode);
    const uint32_t n_parts = (n_blocks + bpu - 1) / bpu;
    ScratchLayout lay(scratch);
    uint8_t *idx_t = lay.take<uint8_t>((size_t)s.n_detectors * pitch);
    uint32_t *part = lay.take<uint32_t>((size_t)n_parts * s.batch * s.n_outputs * 4);
    hipError_t e;
    if (lay.stop(&e, "fill_outputs_fc (table-major)")) return e;
    // the DMA form reads whole 16-byte key pieces: pad the rows with zeros
    const bool dma = std::is_same<WT, float>::value && s.n_entries == (uint32_t)kTmMaxEntries;
    const uint32_t ipitch = dma ? pitch : s.batch;
    const uint64_t grid = (uint64_t)n_parts * n_chunks * n_slices;
    if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_transpose_idx, dim3((s.n_detectors + 63) / 64, (ipitch + 63) / 64),
                       dim3(256), 0, st, idx, idx_t, s.batch, s.n_detectors, ipitch, s.n_entries - 1);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (dma) {
        const float *wf = reinterpret_cast<const float *>(w);
        // a 4-stage ring, one workgroup per CU.  (A 2-stage ring with chunks of
        // 512 samples and two workgroups per CU measured 15% slower at config 3.)
#define SPIKY_TMD(SPT, IM)                                                                         \
    hipLaunchKernelGGL((k_fill_tm_dma<SPT, IM, kDmaRing>), dim3((uint32_t)grid),                   \
                       dim3(kTmThreads), 0, st, wf, idx_t, part, s.batch, ipitch, s.n_outputs,     \
                       s.n_detectors, s.dgs, bpu, n_slices, n_chunks, int_rescaler)
        switch (spt) {
            case 1: if (int_mode) SPIKY_TMD(1, true); else SPIKY_TMD(1, false); break;
            case 2: if (int_mode) SPIKY_TMD(2, true); else SPIKY_TMD(2, false); break;
            case 4: if (int_mode) SPIKY_TMD(4, true); else SPIKY_TMD(4, false); break;
            default: if (int_mode) SPIKY_TMD(8, true); else SPIKY_TMD(8, false); break;
        }
#undef SPIKY_TMD
    } else {
#define SPIKY_TM(SPT, IM)                                                                            \
    hipLaunchKernelGGL((k_fill_tm<SPT, IM, WT>), dim3((uint32_t)grid), dim3(kTmThreads), 0, st, w,  \
                       scales, idx_t, part, s.batch, s.n_outputs, s.n_detectors, s.n_entries, s.dgs, \
                       bpu, n_slices, n_chunks, int_rescaler)
    switch (spt) {
        case 1: if (int_mode) SPIKY_TM(1, true); else SPIKY_TM(1, false); break;
        case 2: if (int_mode) SPIKY_TM(2, true); else SPIKY_TM(2, false); break;
        case 4: if (int_mode) SPIKY_TM(4, true); else SPIKY_TM(4, false); break;
        default: if (int_mode) SPIKY_TM(8, true); else SPIKY_TM(8, false); break;
    }
#undef SPIKY_TM
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint64_t n_quads = (uint64_t)s.batch * s.n_outputs / 4;
    const uint64_t stride = (uint64_t)s.batch * s.n_outputs;
    const uint32_t cgrid = (uint32_t)((n_quads + 255) / 256);
    if (int_mode)
        hipLaunchKernelGGL(k_fill_commit<true>, dim3(cgrid), dim3(256), 0, st, part, out, n_quads,
                           n_parts, stride, int_rescaler);
    else
        hipLaunchKernelGGL(k_fill_commit<false>, dim3(cgrid), dim3(256), 0, st, part, out,
                           n_quads, n_parts, stride, int_rescaler);
    return hipGetLastError();
}

hipError_t launch_fill_tm(const FcShape &s, const float *w, const int32_t *idx, float *out,
                          bool int_mode, double int_rescaler, Scratch &scratch, hipStream_t st) {
    return launch_fill_tm_impl<float>(s, w, nullptr, idx, out, int_mode, int_rescaler, scratch, st);
}

hipError_t launch_fill_tm_i8(const FcShape &s, const int8_t *q8, const float *scales,
                             const int32_t *idx, float *out, bool int_mode, double int_rescaler,
                             Scratch &scratch, hipStream_t st) {
    return launch_fill_tm_impl<int8_t>(s, q8, scales, idx, out, int_mode, int_rescaler, scratch, st);
}

hipError_t launch_block_commit(const uint32_t *part, float *out, uint64_t n, uint32_t n_blocks,
                               bool int_mode, double int_rescaler, hipStream_t st) {
    if (n % 4 != 0) return hipErrorInvalidValue;
    const uint64_t n_quads = n / 4;
    const uint64_t cgrid = (n_quads + 255) / 256;
    if (cgrid > 0x7fffffffu) return hipErrorInvalidConfiguration;
    if (int_mode)
        hipLaunchKernelGGL(k_fill_commit<true>, dim3((uint32_t)cgrid), dim3(256), 0, st, part, out,
                           n_quads, n_blocks, n, int_rescaler);
    else
        hipLaunchKernelGGL(k_fill_commit<false>, dim3((uint32_t)cgrid), dim3(256), 0, st, part, out,
                           n_quads, n_blocks, n, int_rescaler);
    return hipGetLastError();
}

bool tm_propagate_applies(const FcShape &s) {
    const uint64_t n_slices = (s.n_outputs + kTmCols - 1) / kTmCols;
    return s.batch >= 256 && s.n_entries <= (uint32_t)kTmMaxEntries && s.n_outputs % 4 == 0 &&
           s.n_outputs >= 64 && s.n_inputs * 8 <= (uint32_t)kScatterLds &&
           n_slices * s.batch * s.n_detectors * 4 <= (4ull << 30);
}

static hipError_t launch_propagate_finish(const FcShape &s, float *dpart, uint32_t n_slices,
                                          const float *min_deltas, const int32_t *min_idx,
                                          const int32_t *anchors, float *x_grad, hipStream_t st);
static hipError_t launch_propagate_scatter(const FcShape &s, const float *du, const int32_t *min_idx,
                                           const int32_t *anchors, float *x_grad, hipStream_t st);

// the 64-column propagate: whole 256-row fp32 tables, 64-column slices
static bool tm_propagate_wide(const FcShape &s) {
    // k_propagate_units reads g with 32-bit byte offsets, up to a whole chunk
    // past the batch
    return s.n_entries == (uint32_t)kTmMaxEntries && s.n_outputs % 64 == 0 && s.batch >= 256 &&
           (uint64_t)(s.batch + 8 * kUnitPass) * s.n_outputs * 4 <= 0x7fffffffu;
}

uint32_t tm_key_row_shift(const FcShape &s) { return tm_propagate_wide(s) ? 8u : 7u; }

// Samples of a chunk of the whole-table propagate (k_propagate_units): 512 up
// to a batch of 512, else 1024.
static uint32_t tm_units_spt(uint32_t batch) { return batch <= 4u * kUnitPass ? 4u : 8u; }

// Row pitch of the transposed keys: whole chunks of samples of every
// table-major propagate (at least 512 samples, the whole-table kernel's
// smallest chunk), zero past the batch.
uint32_t tm_key_pitch(uint32_t batch) {
    const uint32_t chunk = kTmPass * std::max<uint32_t>(tm_spt(batch), 4u);
    return (batch + chunk - 1) / chunk * chunk;
}

// scratch: keys [T][pitch] u32 | du_t [T][pitch] f32 | then, for the
// whole-table propagate, du [B][T] f32; for the slice propagate, partial dots
// [slices][T][B] f32 and du [B][T] f32 after them
hipError_t launch_propagate_tm(const FcShape &s, const float *w, const float *g,
                               const int32_t *idx, const float *min_deltas,
                               const int32_t *min_idx, const int32_t *anchors, float *x_grad,
                               Scratch &scratch, hipStream_t st) {
    const uint32_t pitch = tm_key_pitch(s.batch);
    const bool wide = tm_propagate_wide(s);
    const uint32_t n_slices = (s.n_outputs + kTmCols - 1) / kTmCols;
    ScratchLayout lay(scratch);
    uint32_t *key_t = lay.take<uint32_t>((size_t)s.n_detectors * pitch * 4);
    float *du_t = lay.take<float>((size_t)s.n_detectors * pitch * 4);
    // wide: du [B][T]; else the slice partials and du after them
    float *dpart = lay.take<float>((size_t)(wide ? 1 : n_slices + 1) * s.batch * s.n_detectors * 4);
    hipError_t e;
    if (lay.stop(&e, "propagate_through_detectors_fc (table-major)")) return e;
    if (s.n_detectors % 4 == 0 && pitch % 4 == 0)
        hipLaunchKernelGGL(k_transpose_keys4, dim3((s.n_detectors + 63) / 64, (pitch + 63) / 64),
                           dim3(256), 0, st, idx, min_idx, min_deltas, key_t, wide ? du_t : nullptr,
                           s.batch, pitch, s.n_detectors, s.n_anchors, s.n_entries, wide ? 8u : 7u);
    else
        hipLaunchKernelGGL(k_transpose_keys, dim3((s.n_detectors + 63) / 64, (pitch + 63) / 64),
                           dim3(256), 0, st, idx, min_idx, min_deltas, key_t, wide ? du_t : nullptr,
                           s.batch, pitch, s.n_detectors, s.n_anchors, s.n_entries, wide ? 8u : 7u);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t tpu = 32;
    const uint32_t n_units = (s.n_detectors + tpu - 1) / tpu;
    if (wide) {
        // whole tables, every 64-column slice in one unit: du[b][t] directly
        // 8 tables a unit.  g is read once per unit and slice, so 16 tables
        // halve its reads and ran 1.56 against 1.59 ms at config 3, but their
        // keys and du (8 KiB a table, read again for every slice) then
        // overflow an XCD's L2 and the kernel fetches 9.73 instead of 8.80 GB;
        // 12 leaves a partial last round of units (1.75 ms)
        // Few tables over many samples (a transformer's feed-forward layer: 16
        // tables, 8192 rows) would leave most CUs idle at 8 tables a unit: fewer
        // tables a unit then, down to one, until the grid covers the 256 CUs.
        const uint32_t spt = tm_units_spt(s.batch);
        const uint32_t n_chunks = (s.batch + kUnitPass * spt - 1) / (kUnitPass * spt);
        uint32_t tpu = 8;
        while (tpu > 1 && (uint64_t)((s.n_detectors + tpu - 1) / tpu) * n_chunks < 256) tpu /= 2;
        const uint64_t grid = (uint64_t)((s.n_detectors + tpu - 1) / tpu) * n_chunks;
        if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
        float *du = dpart;
#define SPIKY_PU(SPT, TPU)                                                                          \
    hipLaunchKernelGGL((k_propagate_units<SPT, TPU>), dim3((uint32_t)grid), dim3(kTmThreads), 0, st, w, g, \
                       key_t, du_t, du, s.batch, pitch, s.n_outputs, s.n_detectors, n_chunks,            \
                       s.ogs == (uint32_t)kTmCols)
#define SPIKY_PU_T(SPT)                    \
    switch (tpu) {                         \
        case 1: SPIKY_PU(SPT, 1); break;   \
        case 2: SPIKY_PU(SPT, 2); break;   \
        case 4: SPIKY_PU(SPT, 4); break;   \
        default: SPIKY_PU(SPT, 8); break;  \
    }
        if (spt == 4) {
            SPIKY_PU_T(4)
        } else {
            SPIKY_PU_T(8)
        }
#undef SPIKY_PU_T
#undef SPIKY_PU
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_propagate_scatter(s, du, min_idx, anchors, x_grad, st);
    }
    // the LDS-DMA ring needs whole 256-row tables
    const bool dma = s.n_entries == (uint32_t)kTmMaxEntries;
    const uint32_t spt = tm_spt(s.batch);
    const uint32_t n_chunks = (s.batch + kTmPass * spt - 1) / (kTmPass * spt);
    const uint64_t grid = (uint64_t)n_units * n_chunks * n_slices;
    if (grid > 0x7fffffffu) return hipErrorInvalidConfiguration;
#define SPIKY_PTM(SPT)                                                                              \
    if (dma)                                                                                        \
        hipLaunchKernelGGL((k_propagate_tm_dma<SPT, kDmaRing>), dim3((uint32_t)grid),              \
                           dim3(kTmThreads), 0, st,                                                 \
                           w, g, key_t, dpart, s.batch, pitch, s.n_outputs, s.n_detectors, tpu,   \
                           n_slices, n_chunks);                                                    \
    else                                                                                            \
        hipLaunchKernelGGL((k_propagate_tm<SPT>), dim3((uint32_t)grid), dim3(kTmThreads), 0, st, w, \
                           g, key_t, dpart, s.batch, pitch, s.n_outputs, s.n_detectors,            \
                           s.n_entries, tpu, n_slices, n_chunks)
    switch (spt) {
        case 1: SPIKY_PTM(1); break;
        case 2: SPIKY_PTM(2); break;
        case 4: SPIKY_PTM(4); break;
        default: SPIKY_PTM(8); break;
    }
#undef SPIKY_PTM
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_propagate_finish(s, dpart, n_slices, min_deltas, min_idx, anchors, x_grad, st);
}

// du from the slice partials, then the input-gradient scatter
static hipError_t launch_propagate_finish(const FcShape &s, float *dpart, uint32_t n_slices,
                                          const float *min_deltas, const int32_t *min_idx,
                                          const int32_t *anchors, float *x_grad, hipStream_t st) {
    hipError_t e;
    float *du = dpart + (size_t)n_slices * s.batch * s.n_detectors;
    hipLaunchKernelGGL(k_propagate_reduce, dim3((s.n_detectors + 63) / 64, (s.batch + 63) / 64),
                       dim3(256), 0, st, dpart, min_deltas, min_idx, du, s.batch, s.n_detectors,
                       s.n_anchors, n_slices, s.ogs == (uint32_t)kTmCols);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_propagate_scatter(s, du, min_idx, anchors, x_grad, st);
}

// x_grad from du [B][T]
static hipError_t launch_propagate_scatter(const FcShape &s, const float *du, const int32_t *min_idx,
                                           const int32_t *anchors, float *x_grad, hipStream_t st) {
    const uint32_t spg = std::max<uint32_t>(1, std::min<uint32_t>(16, kScatterLds / 8 / s.n_inputs));
    const uint32_t groups = (s.batch + spg - 1) / spg;
    hipLaunchKernelGGL(k_propagate_scatter, dim3(groups), dim3(kScatterThreads), 0, st, du,
                       min_idx, reinterpret_cast<const int2 *>(anchors), x_grad, s.batch,
                       s.n_inputs, s.n_detectors, s.n_anchors, spg);
    return hipGetLastError();
}

}  // namespace spiky
