// lut_densify.hip -- dense -> sparse (COO) compaction of 32-bit tensors for
// gfx950: the GradientType.Sparse weight-gradient export.
//
// It replaces the reference's DenseToSparseConverterNative
// (spiky_cuda/torch_utils/torch_utils.cu:11-339, densify_logic /
// densify_new_logic in torch_utils_kernels_logic.proto:1-324) with the same
// element test -- a 32-bit word is kept when its bit pattern is non-zero, so a
// float -0.0 is kept, as in the reference's int4 compare -- and the same
// outputs: int64 element indices and the raw 32-bit values, optionally zeroing
// the kept words of the source.  The reference orders its output only within
// a block (blocks claim their output range with an atomic); here the ranges
// come from a scan over tiles, so the output is in ascending index order and
// identical from run to run.
//
// Passes over tiles of kDzTileQuads 16-byte quads (thread t of a tile owns
// quads j * 256 + t, j < 4: each load instruction reads 4 KiB contiguously):
//   k_dz_count        nonzero words per tile                     (reads the source)
//   k_dz_scan_chunks  exclusive scan of the tile counts within chunks of 1024
//                     tiles (one workgroup each), chunk totals
//   k_dz_scan_top     exclusive scan of the chunk totals, grand total
//   k_dz_write        each tile re-tests its quads and writes its words at
//                     chunk offset + tile offset, ascending; erases kept words
// The bound is HBM: 4 bytes per element read twice, 12 bytes per kept word
// written (plus 16 per erased quad).
#include "lut_kernels.h"

namespace spiky {
namespace {

constexpr int kDzThreads = 256;
constexpr int kDzQuadsPerThread = 4;
constexpr uint32_t kDzTileQuads = kDzThreads * kDzQuadsPerThread;
constexpr int kDzScanThreads = 1024;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t quad_mask(u32x4 v) {
    return (uint32_t)(v.x != 0u) | ((uint32_t)(v.y != 0u) << 1) | ((uint32_t)(v.z != 0u) << 2) |
           ((uint32_t)(v.w != 0u) << 3);
}

// Inclusive scan over the 64 lanes of a wavefront.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, uint32_t lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(v, off, 64);
        if (lane >= (uint32_t)off) v += y;
    }
    return v;
}

__global__ __launch_bounds__(kDzThreads) void k_dz_count(const u32x4 *__restrict__ src,
                                                         uint64_t n_quads,
                                                         uint32_t *__restrict__ counts) {
    __shared__ uint32_t wsum[kDzThreads / 64];
    const uint32_t tid = threadIdx.x;
    const uint64_t q0 = (uint64_t)blockIdx.x * kDzTileQuads + tid;
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < kDzQuadsPerThread; j++) {
        const uint64_t qi = q0 + (uint64_t)j * kDzThreads;
        if (qi < n_quads) c += __popc(quad_mask(src[qi]));
    }
    const uint32_t lane = tid & 63;
    const uint32_t incl = wave_incl_scan(c, lane);
    if (lane == 63) wsum[tid / 64] = incl;
    __syncthreads();
    if (tid == 0) {
        uint32_t t = 0;
#pragma unroll
        for (int w = 0; w < kDzThreads / 64; w++) t += wsum[w];
        counts[blockIdx.x] = t;
    }
}

// Block-wide exclusive scan of one value per thread (kDzScanThreads); returns
// the exclusive prefix and sets *all to the block total.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *wsum, uint32_t *all) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid / 64;
    const uint32_t incl = wave_incl_scan(v, lane);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    uint32_t before = 0, tot = 0;
    for (uint32_t w = 0; w < blockDim.x / 64; w++) {
        const uint32_t s = wsum[w];
        if (w < wave) before += s;
        tot += s;
    }
    *all = tot;
    return before + incl - v;
}

// counts[i] -> exclusive prefix within its chunk of kDzScanThreads tiles;
// chunk_tot[c] = the chunk's total.
__global__ __launch_bounds__(kDzScanThreads) void k_dz_scan_chunks(uint32_t *__restrict__ counts,
                                                                   uint64_t n_tiles,
                                                                   uint64_t *__restrict__ chunk_tot) {
    __shared__ uint32_t wsum[kDzScanThreads / 64];
    const uint64_t i = (uint64_t)blockIdx.x * kDzScanThreads + threadIdx.x;
    const uint32_t v = i < n_tiles ? counts[i] : 0u;
    uint32_t all;
    const uint32_t ex = block_excl_scan(v, wsum, &all);
    if (i < n_tiles) counts[i] = ex;
    if (threadIdx.x == 0) chunk_tot[blockIdx.x] = all;
}

// chunk_tot[c] -> exclusive prefix over chunks (in place), *total = the sum.
__global__ __launch_bounds__(kDzScanThreads) void k_dz_scan_top(uint64_t *__restrict__ chunk_tot,
                                                                uint64_t n_chunks,
                                                                int64_t *__restrict__ total) {
    __shared__ uint64_t wsum[kDzScanThreads / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint64_t per = (n_chunks + kDzScanThreads - 1) / kDzScanThreads;
    const uint64_t i0 = min((uint64_t)tid * per, n_chunks);
    const uint64_t i1 = min(i0 + per, n_chunks);
    uint64_t local = 0;
    for (uint64_t i = i0; i < i1; i++) local += chunk_tot[i];
    uint64_t incl = local;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t y = __shfl_up(incl, off, 64);
        if (lane >= (uint32_t)off) incl += y;
    }
    if (lane == 63) wsum[tid / 64] = incl;
    __syncthreads();
    uint64_t run = incl - local;
    for (uint32_t w = 0; w < tid / 64; w++) run += wsum[w];
    for (uint64_t i = i0; i < i1; i++) {
        const uint64_t c = chunk_tot[i];
        chunk_tot[i] = run;
        run += c;
    }
    if (tid == kDzScanThreads - 1) *total = (int64_t)run;
}

// In index order, quad j of every thread precedes quad j + 1 of every thread.
// The four per-thread counts are scanned at once as 16-bit fields of a u64
// (a tile holds at most 4096 words, so no field overflows).
__global__ __launch_bounds__(kDzThreads) void k_dz_write(u32x4 *__restrict__ src, uint64_t n_quads,
                                                         const uint32_t *__restrict__ tile_off,
                                                         const uint64_t *__restrict__ chunk_off,
                                                         int64_t *__restrict__ indices,
                                                         uint32_t *__restrict__ values,
                                                         uint64_t capacity, bool erase) {
    __shared__ uint64_t wsum[kDzThreads / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid / 64;
    const uint64_t q0 = (uint64_t)blockIdx.x * kDzTileQuads + tid;
    u32x4 v[kDzQuadsPerThread];
    uint32_t m[kDzQuadsPerThread];
    uint64_t packed = 0;
#pragma unroll
    for (int j = 0; j < kDzQuadsPerThread; j++) {
        const uint64_t qi = q0 + (uint64_t)j * kDzThreads;
        v[j] = (qi < n_quads) ? src[qi] : u32x4{0u, 0u, 0u, 0u};
        m[j] = quad_mask(v[j]);
        packed |= (uint64_t)__popc(m[j]) << (16 * j);
    }
    uint64_t incl = packed;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t y = __shfl_up(incl, off, 64);
        if (lane >= (uint32_t)off) incl += y;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    uint64_t before = incl - packed, all = 0;
#pragma unroll
    for (int w = 0; w < kDzThreads / 64; w++) {
        const uint64_t sw = wsum[w];
        if ((uint32_t)w < wave) before += sw;
        all += sw;
    }
    const uint64_t base = chunk_off[blockIdx.x / kDzScanThreads] + tile_off[blockIdx.x];
    uint64_t jbase = base;
#pragma unroll
    for (int j = 0; j < kDzQuadsPerThread; j++) {
        uint64_t pos = jbase + ((before >> (16 * j)) & 0xFFFFu);
        jbase += (all >> (16 * j)) & 0xFFFFu;
        if (!m[j]) continue;
        const uint64_t qi = q0 + (uint64_t)j * kDzThreads;
        const uint32_t vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            if ((m[j] >> e) & 1u) {
                if (pos < capacity) {
                    indices[pos] = (int64_t)(qi * 4 + (uint64_t)e);
                    values[pos] = vv[e];
                }
                pos++;
            }
        }
        if (erase) src[qi] = u32x4{0u, 0u, 0u, 0u};
    }
}

uint64_t dz_tiles(uint64_t n) { return (n / 4 + kDzTileQuads - 1) / kDzTileQuads; }
uint64_t dz_chunks(uint64_t n_tiles) { return (n_tiles + kDzScanThreads - 1) / kDzScanThreads; }

}  // namespace

// workspace: tile offsets u32 [n_tiles] (8-byte padded) | chunk offsets u64 [n_chunks]
uint64_t densify32_workspace_bytes(uint64_t n) {
    const uint64_t t = dz_tiles(n);
    return ((t * 4 + 7) & ~(uint64_t)7) + (dz_chunks(t) + 1) * 8;
}

hipError_t launch_densify32_count(const uint32_t *src, uint64_t n, void *workspace,
                                  int64_t *total, hipStream_t st) {
    const uint64_t n_tiles = dz_tiles(n);
    const uint64_t n_chunks = dz_chunks(n_tiles);
    if (n_tiles > 0x7fffffffu) return hipErrorInvalidConfiguration;
    uint32_t *counts = reinterpret_cast<uint32_t *>(workspace);
    uint64_t *chunk = reinterpret_cast<uint64_t *>(reinterpret_cast<uint8_t *>(workspace) +
                                                   ((n_tiles * 4 + 7) & ~(uint64_t)7));
    if (n_tiles > 0) {
        hipLaunchKernelGGL(k_dz_count, dim3((uint32_t)n_tiles), dim3(kDzThreads), 0, st,
                           reinterpret_cast<const u32x4 *>(src), n / 4, counts);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(k_dz_scan_chunks, dim3((uint32_t)n_chunks), dim3(kDzScanThreads), 0, st,
                           counts, n_tiles, chunk);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k_dz_scan_top, dim3(1), dim3(kDzScanThreads), 0, st, chunk, n_chunks, total);
    return hipGetLastError();
}

hipError_t launch_densify32_write(uint32_t *src, uint64_t n, const void *workspace,
                                  int64_t *indices, uint32_t *values, uint64_t capacity, bool erase,
                                  hipStream_t st) {
    const uint64_t n_tiles = dz_tiles(n);
    if (n_tiles == 0) return hipSuccess;
    if (n_tiles > 0x7fffffffu) return hipErrorInvalidConfiguration;
    const uint32_t *tile_off = reinterpret_cast<const uint32_t *>(workspace);
    const uint64_t *chunk_off = reinterpret_cast<const uint64_t *>(
        reinterpret_cast<const uint8_t *>(workspace) + ((n_tiles * 4 + 7) & ~(uint64_t)7));
    hipLaunchKernelGGL(k_dz_write, dim3((uint32_t)n_tiles), dim3(kDzThreads), 0, st,
                       reinterpret_cast<u32x4 *>(src), n / 4, tile_off, chunk_off, indices, values,
                       capacity, erase);
    return hipGetLastError();
}

}  // namespace spiky
