// lut_product.hip -- product mode (concatenation_product == False) of the
// sequence LUT layer for gfx950.
//
// Every causal pair i < j of a sequence is one lookup of each table t over the
// virtual input row [x1[i] | x2[j] | pe[j-i-1][t]] (sliced mode: the
// interleaving x1[0] x2[0] pe[0] x1[1] ...), reference
// calculate_product_lookup_index(_backprop) (lut_runtime_kernels_logic.proto:
// 32-181), fill_outputs_product_cpu_logic (proto:2148-2264) and
// propagate_backward_product_cpu_logic (proto:2396-2628).
//
// The reference gathers one table row per (pair, table) -- S^2/2 * T rows of O
// floats per sequence.  Here the pairs are reduced to counts first:
// Cnt[b*S + j][t*E + e] = #{i < j : pair (i, j) of table t looks up row e}.
// Then
//   forward            out  (+)= Cnt . W                  (M = B*S, K = T*E)
//   backward  sums     P     =   G . W^T  (fp64)         (the pairs' main and
//                      alternative sums are P[bj][t*E + idx], P[bj][t*E + alt])
//             weights  target (+)= Cnt^T . g'             g' = g*lr where |g| > EPS
// and one pass over the pairs forms du from P and pushes it to the two
// inputs of the min-margin anchor.  The products run on the VALU in fp64
// (int32 summation: wrapping int32, which is exact and order-free, as in the
// reference); they are small next to the pair enumeration at these shapes.
//
// Parity: int32 summation is bit-exact (every term is the reference's
// payload, and wrapping int32 sums do not depend on order).  fp32 outputs and
// gradients are fp64 sums rounded once, where the reference adds fp32 terms
// in a serial order: equal within the fp32 rounding of that order.
#include "lut_kernels.h"

#include <type_traits>

namespace spiky {
namespace {

constexpr int kPrThreads = 256;
constexpr uint32_t kPrMaxHist = 16384;  // T * E counters per (b, j) in LDS

__device__ __forceinline__ double du_of_margin(float md) {
    double du = (double)md;
    double r = 1.0 / (1.0 + fabs(du));
    return (du > 0) ? r * (0.5 * r) : r * (-0.5 * r);
}

// ROUNDED_COMPARISON_GREATER(delta, 0.0, cmp_eps), misc.h:16
__device__ __forceinline__ bool rgreater0(float d, float cmp_eps) {
    if (cmp_eps == 0.0f) return d > 0.0f;
    return (fabsf(d) < cmp_eps) ? false : (d > 0.0f);
}

struct PairLookup {
    int32_t idx, alt;
    float md;
    int32_t src1, src2;  // 0: x1[i], 1: x2[j], 2: pe; -1: no valid anchor
    uint32_t k1, k2;
};

// Where virtual input `id` lives; false when it is beyond the row (such an
// anchor is skipped like an unused one, so no lookup reads out of bounds).
__device__ __forceinline__ bool prod_locate(uint32_t n1, uint32_t n2, uint32_t pd, bool sliced,
                                            uint32_t id, int32_t &src, uint32_t &k) {
    if (sliced) {
        src = (int32_t)(id % 3);
        k = id / 3;
    } else if (id < n1) {
        src = 0;
        k = id;
    } else if (id < n1 + n2) {
        src = 1;
        k = id - n1;
    } else {
        src = 2;
        k = id - n1 - n2;
    }
    return k < (src == 0 ? n1 : (src == 1 ? n2 : pd));
}

__device__ __forceinline__ float prod_value(const float *x1i, const float *x2j, const float *pet,
                                            int32_t src, uint32_t k) {
    return src == 0 ? x1i[k] : (src == 1 ? x2j[k] : pet[k]);
}

// Lookup index, and the min-margin anchor (strict |d| < |min| from FLT_MAX:
// the first of equal margins wins), proto:102-181.
__device__ __forceinline__ PairLookup prod_lookup(const float *x1i, const float *x2j,
                                                  const float *pet, const int2 *anc,
                                                  uint32_t n_anchors, uint32_t n1, uint32_t n2,
                                                  uint32_t pd, bool sliced, float cmp_eps) {
    PairLookup p;
    p.idx = 0;
    p.md = 3.402823466e+38f;
    p.src1 = p.src2 = -1;
    p.k1 = p.k2 = 0;
    int32_t flip = -1;
    for (uint32_t a = 0; a < n_anchors; a++) {
        const int2 ap = anc[a];
        if (ap.x < 0 || ap.y < 0) continue;  // unused pair
        int32_t s1, s2;
        uint32_t i1, i2;
        if (!prod_locate(n1, n2, pd, sliced, (uint32_t)ap.x, s1, i1) ||
            !prod_locate(n1, n2, pd, sliced, (uint32_t)ap.y, s2, i2))
            continue;
        const float v1 = prod_value(x1i, x2j, pet, s1, i1);
        const float v2 = prod_value(x1i, x2j, pet, s2, i2);
        const float d = v1 - v2;
        if (rgreater0(d, cmp_eps)) p.idx |= (1 << a);
        if (fabsf(d) < fabsf(p.md)) {
            p.md = d;
            flip = (int32_t)a;
            p.src1 = s1;
            p.src2 = s2;
            p.k1 = i1;
            p.k2 = i2;
        }
    }
    p.alt = flip >= 0 ? (p.idx ^ (1 << flip)) : p.idx;
    return p;
}

// One workgroup per (b, j): every pair (t, i < j) is looked up; the counts
// of (t, row) go through an LDS histogram to cnt[b*S + j][t*E + e] (fp32,
// exact small integers).  BWD additionally forms du from P and pushes it.
template <bool BWD, bool INT_MODE>
__global__ __launch_bounds__(kPrThreads) void k_prod_pairs(
    const float *__restrict__ x1, const float *__restrict__ x2, const float *__restrict__ pe,
    const int2 *__restrict__ anchors, const double *__restrict__ P, float *__restrict__ cnt,
    float *__restrict__ x1_grad, float *__restrict__ x2_grad, float *__restrict__ pe_grad,
    uint32_t S, uint32_t n1, uint32_t n2, uint32_t pd, uint32_t T, uint32_t n_anchors, bool sliced,
    float cmp_eps, double int_rescaler) {
    extern __shared__ uint32_t hist[];  // T * E counters
    const uint32_t E = 1u << n_anchors;
    const uint32_t TE = T * E;
    const uint32_t bj = blockIdx.x;
    const uint32_t b = bj / S, j = bj % S;
    for (uint32_t k = threadIdx.x; k < TE; k += kPrThreads) hist[k] = 0;
    __syncthreads();
    const float *x2j = x2 + (size_t)bj * n2;
    const double *Pbj = BWD ? P + (size_t)bj * TE : nullptr;
    const uint32_t n_pairs = T * j;
    for (uint32_t p = threadIdx.x; p < n_pairs; p += kPrThreads) {
        const uint32_t t = p / j, i = p % j;
        const float *x1i = x1 + ((size_t)b * S + i) * n1;
        const size_t pe_off = ((size_t)(j - i - 1) * T + t) * pd;
        const PairLookup lk = prod_lookup(x1i, x2j, pd ? pe + pe_off : nullptr,
                                          anchors + (size_t)t * n_anchors, n_anchors, n1, n2,
                                          pd, sliced, cmp_eps);
        atomicAdd(&hist[t * E + (uint32_t)lk.idx], 1u);
        if (BWD && lk.src1 >= 0) {
            const double du = du_of_margin(lk.md) * (Pbj[t * E + lk.idx] - Pbj[t * E + lk.alt]);
            if (fabs(du) > kEps) {
                float *dst[3] = {x1_grad + ((size_t)b * S + i) * n1, x2_grad + (size_t)bj * n2,
                                 pd ? pe_grad + pe_off : nullptr};
                const int32_t srcs[2] = {lk.src1, lk.src2};
                const uint32_t ks[2] = {lk.k1, lk.k2};
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    float *d = dst[srcs[h]];
                    if (!d) continue;
                    const double v = h == 0 ? du : -du;
                    if (INT_MODE)
                        atomicAdd(reinterpret_cast<int32_t *>(d + ks[h]),
                                  (int32_t)(v * kDenom32 * int_rescaler));
                    else
                        atomicAdd(d + ks[h], (float)v);
                }
            }
        }
    }
    __syncthreads();
    float *crow = cnt + (size_t)bj * TE;
    for (uint32_t k = threadIdx.x; k < TE; k += kPrThreads) crow[k] = (float)hist[k];
}

// C[M][N] (+)= A[M][K] . B[K][N] on the VALU: 64 x 64 tiles, 256 threads of 4 x 4
// outputs, K in steps of 16 through LDS.  A(m, k) = TA ? A[k*lda + m] : A[m*lda + k],
// B likewise with TB.  BMODE: 0 plain; 1 weight payload (int32 forward); 2 weight-
// gradient term g*lr where |g| > EPS (or its int32 payload).  OUT: 0 fp32 +=,
// 1 int32 wrapping += on the fp32 buffer's bits, 2 fp64 store.
constexpr int kGmTile = 64;
constexpr int kGmK = 16;

template <bool TA, bool TB, int BMODE, int OUT>
__global__ __launch_bounds__(256) void k_prod_gemm(const float *__restrict__ A, uint32_t lda,
                                                   const float *__restrict__ B, uint32_t ldb,
                                                   void *__restrict__ C, uint32_t M, uint32_t N,
                                                   uint32_t K, double lr, double int_rescaler) {
    constexpr bool INT = OUT == 1;
    typedef typename std::conditional<INT, uint32_t, double>::type acc_t;
    __shared__ acc_t As[kGmK][kGmTile + 1];
    __shared__ acc_t Bs[kGmK][kGmTile + 1];
    const uint32_t tid = threadIdx.x;
    const uint32_t tx = tid & 15, ty = tid >> 4;
    const uint32_t m0 = blockIdx.y * kGmTile, n0 = blockIdx.x * kGmTile;
    acc_t acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[r][c] = 0;
    for (uint32_t k0 = 0; k0 < K; k0 += kGmK) {
        // 1024 elements of each tile, 4 per thread; the index order follows
        // the contiguous dimension of the source for coalescing
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t e = tid + 256u * u;
            uint32_t kk, mm;
            if (TA) { mm = e & 63; kk = e >> 6; } else { kk = e & 15; mm = e >> 4; }
            const uint32_t m = m0 + mm, k = k0 + kk;
            float a = 0.0f;
            if (m < M && k < K) a = TA ? A[(size_t)k * lda + m] : A[(size_t)m * lda + k];
            As[kk][mm] = INT ? (acc_t)(uint32_t)a : (acc_t)a;
            uint32_t kb, nn;
            if (TB) { kb = e & 15; nn = e >> 4; } else { nn = e & 63; kb = e >> 6; }
            const uint32_t n = n0 + nn, k2 = k0 + kb;
            float bv = 0.0f;
            if (n < N && k2 < K) bv = TB ? B[(size_t)n * ldb + k2] : B[(size_t)k2 * ldb + n];
            acc_t bt;
            if (BMODE == 0) {
                bt = INT ? (acc_t)(uint32_t)(int32_t)bv : (acc_t)bv;
            } else if (BMODE == 1) {
                bt = (acc_t)(uint32_t)(int32_t)((double)bv * kDenom32 * int_rescaler);
            } else {
                const double gg = (double)bv;
                if (!(fabs(gg) > kEps)) bt = 0;
                else if (INT) bt = (acc_t)(uint32_t)(int32_t)(gg * lr * kDenom32 * int_rescaler);
                else bt = (acc_t)(gg * lr);
            }
            Bs[kb][nn] = bt;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kGmK; kk++) {
            acc_t a[4], bb[4];
#pragma unroll
            for (int r = 0; r < 4; r++) a[r] = As[kk][ty * 4 + r];
#pragma unroll
            for (int c = 0; c < 4; c++) bb[c] = Bs[kk][tx * 4 + c];
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int c = 0; c < 4; c++) acc[r][c] += a[r] * bb[c];
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t m = m0 + ty * 4 + r;
        if (m >= M) continue;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t n = n0 + tx * 4 + c;
            if (n >= N) continue;
            const size_t o = (size_t)m * N + n;
            if (OUT == 0) {
                float *Cf = reinterpret_cast<float *>(C);
                Cf[o] = (float)((double)Cf[o] + (double)acc[r][c]);
            } else if (OUT == 1) {
                uint32_t *Ci = reinterpret_cast<uint32_t *>(C);
                Ci[o] = Ci[o] + (uint32_t)acc[r][c];
            } else {
                reinterpret_cast<double *>(C)[o] = (double)acc[r][c];
            }
        }
    }
}

template <bool TA, bool TB, int BMODE, int OUT>
hipError_t gemm(const float *A, uint32_t lda, const float *B, uint32_t ldb, void *C, uint32_t M,
                uint32_t N, uint32_t K, double lr, double int_rescaler, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    const dim3 grid((N + kGmTile - 1) / kGmTile, (M + kGmTile - 1) / kGmTile);
    if (grid.y > 65535u) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((k_prod_gemm<TA, TB, BMODE, OUT>), grid, dim3(256), 0, st, A, lda, B, ldb, C,
                       M, N, K, lr, int_rescaler);
    return hipGetLastError();
}

}  // namespace

bool product_applies(const ProductShape &s) {
    const uint64_t TE = (uint64_t)s.n_detectors << s.n_anchors;
    return s.n_anchors <= 16 && TE <= kPrMaxHist && (uint64_t)s.batch * s.seq_len <= 0x7fffffffu &&
           (uint64_t)s.batch * s.seq_len <= 65535ull * kGmTile;
}

// scratch: Cnt [B*S][T*E] f32 | P [B*S][T*E] f64 (backward)
size_t product_scratch_bytes(const ProductShape &s, bool backward) {
    const uint64_t TE = (uint64_t)s.n_detectors << s.n_anchors;
    const uint64_t BS = (uint64_t)s.batch * s.seq_len;
    const size_t cnt = (BS * TE * 4 + 255) & ~(size_t)255;
    return cnt + (backward ? BS * TE * 8 : 0);
}

hipError_t launch_forward_product(const ProductShape &s, const float *w, const float *x1,
                                  const float *x2, const float *pe, const int32_t *anchors,
                                  float *out, bool int_mode, double int_rescaler, void *scratch,
                                  hipStream_t st) {
    const uint32_t E = 1u << s.n_anchors;
    const uint32_t TE = s.n_detectors * E;
    const uint32_t BS = s.batch * s.seq_len;
    if (BS == 0) return hipSuccess;
    float *cnt = reinterpret_cast<float *>(scratch);
    const int2 *anc = reinterpret_cast<const int2 *>(anchors);
#define SPIKY_PP(IM)                                                                              \
    hipLaunchKernelGGL((k_prod_pairs<false, IM>), dim3(BS), dim3(kPrThreads), TE * 4, st, x1, x2, \
                       pe, anc, (const double *)nullptr, cnt, (float *)nullptr, (float *)nullptr, \
                       (float *)nullptr, s.seq_len, s.n1, s.n2, s.pd, s.n_detectors, s.n_anchors, \
                       s.sliced, s.cmp_eps, int_rescaler)
    if (int_mode) SPIKY_PP(true); else SPIKY_PP(false);
#undef SPIKY_PP
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // out[bj][o] (+)= sum_k cnt[bj][k] * W[k][o]
    if (int_mode)
        return gemm<false, false, 1, 1>(cnt, TE, w, s.n_outputs, out, BS, s.n_outputs, TE, 0.0,
                                        int_rescaler, st);
    return gemm<false, false, 0, 0>(cnt, TE, w, s.n_outputs, out, BS, s.n_outputs, TE, 0.0,
                                    int_rescaler, st);
}

hipError_t launch_backward_product(const ProductShape &s, const float *w, const float *x1,
                                   const float *x2, const float *pe, const int32_t *anchors,
                                   const float *g, float *x1_grad, float *x2_grad, float *pe_grad,
                                   float *target, double lr, bool int_mode, double int_rescaler,
                                   void *scratch, hipStream_t st) {
    const uint32_t E = 1u << s.n_anchors;
    const uint32_t TE = s.n_detectors * E;
    const uint32_t BS = s.batch * s.seq_len;
    if (BS == 0) return hipSuccess;
    float *cnt = reinterpret_cast<float *>(scratch);
    double *P = reinterpret_cast<double *>(reinterpret_cast<uint8_t *>(scratch) +
                                           (((size_t)BS * TE * 4 + 255) & ~(size_t)255));
    // P[bj][k] = sum_o g[bj][o] * W[k][o]  (fp64)
    hipError_t e = gemm<false, true, 0, 2>(g, s.n_outputs, w, s.n_outputs, P, BS, TE, s.n_outputs,
                                           0.0, int_rescaler, st);
    if (e != hipSuccess) return e;
    const int2 *anc = reinterpret_cast<const int2 *>(anchors);
#define SPIKY_PB(IM)                                                                              \
    hipLaunchKernelGGL((k_prod_pairs<true, IM>), dim3(BS), dim3(kPrThreads), TE * 4, st, x1, x2,   \
                       pe, anc, P, cnt, x1_grad, x2_grad, pe_grad, s.seq_len, s.n1, s.n2, s.pd,  \
                       s.n_detectors, s.n_anchors, s.sliced, s.cmp_eps, int_rescaler)
    if (int_mode) SPIKY_PB(true); else SPIKY_PB(false);
#undef SPIKY_PB
    e = hipGetLastError();
    if (e != hipSuccess || target == nullptr) return e;
    // target[k][o] (+)= sum_bj cnt[bj][k] * g'[bj][o]
    if (int_mode)
        return gemm<true, false, 2, 1>(cnt, TE, g, s.n_outputs, target, TE, s.n_outputs, BS, lr,
                                       int_rescaler, st);
    return gemm<true, false, 2, 0>(cnt, TE, g, s.n_outputs, target, TE, s.n_outputs, BS, lr,
                                   int_rescaler, st);
}

}  // namespace spiky
