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

#include <algorithm>
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

// Table-major pass: one workgroup of 1024 threads per (b, table t, block of
// JB positions j).  Every lane looks up the same table, so the only inputs it
// reads are the 2*Nc anchor inputs of t, staged once per row, slot-major:
//   code [Nc]      int2   the two operands of each anchor: source (x1[b, i],
//                          x2[b, j] or pe[j-i-1]) << 28 | slot * R; -1 = unused
//   hist [JB*E/2]  u32    counts of (j, row e), two 16-bit counters a word
//                          (a count is at most S - 1 < 65536)
//   xs   [2Nc][R]  f32    value of slot s in row r (R = last j of the block + 1)
//   acc  [2Nc][R]  f32    (BWD) pushes into slot s of row r, flushed once
// Pairs go j-major over the lanes, so a wave reads consecutive rows i of a
// slot (conflict-free) and one row j (a broadcast).  P is read from L2: the
// lanes of a wave share j, so each read touches a few lines of one 8*E-byte
// row segment.  Pushes into rows i and distances j-i-1 are LDS atomics on
// consecutive words; pushes into the shared row j are summed over the wave
// first (one atomic per slot), since up to 64 lanes would hit one word.
// fp32 pushes are summed in fp64 LDS words: on gfx950 ds_add_f64 sustains
// about 7.5 lanes a clock per CU on consecutive words, ds_add_f32 0.33.
// Pushes reach HBM as one atomic per (row, slot) per workgroup.
constexpr uint32_t kTbThreads = 1024;
constexpr uint32_t kPtBudget = 80 * 1024;  // two workgroups a CU

struct TableLayout {
    uint32_t jb;  // positions per workgroup; 0 = does not fit
    uint32_t bytes;
};

// LDS: anchor codes (8 B each), the packed histogram (rounded up to 8 B), the
// slot values (4 B), and in the backward the push sums (acc_bytes each).
TableLayout table_layout(const ProductShape &s, bool bwd, uint32_t acc_bytes) {
    const uint64_t E = 1ull << s.n_anchors;
    const uint64_t NS = 2ull * s.n_anchors;
    const uint64_t fixed = (uint64_t)s.n_anchors * 8 + 4 + (uint64_t)s.seq_len * NS * (4 + (bwd ? acc_bytes : 0));
    const uint64_t per_j = E * 2;
    if (fixed + per_j > kPtBudget || NS * s.seq_len >= (1ull << 28)) return {0, 0};
    uint64_t jb = (kPtBudget - fixed) / per_j;
    if (jb > s.seq_len) jb = s.seq_len;
    return {(uint32_t)jb, (uint32_t)(fixed + ((jb * E + 1) / 2) * 4)};
}

// The grid is one dimension of B * T * ceil(S / JB) workgroups.
TableLayout table_grid_ok(const ProductShape &s, TableLayout lay) {
    if (!lay.jb) return lay;
    const uint64_t n = (uint64_t)s.batch * s.n_detectors * ((s.seq_len + lay.jb - 1) / lay.jb);
    return n <= 0x7fffffffull ? lay : TableLayout{0, 0};
}

// Sum over the 64 lanes of a wave (every lane active): rotations within rows
// of 16, then the four row sums.
template <typename V>
__device__ __forceinline__ V wave_sum64(V v) {
    auto rot = [](V x, auto ctrl) {
        int xi;
        __builtin_memcpy(&xi, &x, 4);
        xi = __builtin_amdgcn_mov_dpp(xi, decltype(ctrl)::value, 0xF, 0xF, false);
        V r;
        __builtin_memcpy(&r, &xi, 4);
        return r;
    };
    v += rot(v, std::integral_constant<int, 0x128>{});  // row_ror:8
    v += rot(v, std::integral_constant<int, 0x124>{});  // row_ror:4
    v += rot(v, std::integral_constant<int, 0x122>{});  // row_ror:2
    v += rot(v, std::integral_constant<int, 0x121>{});  // row_ror:1
    int vi;
    __builtin_memcpy(&vi, &v, 4);
    V r0, r1, r2, r3;
    int t0 = __builtin_amdgcn_readlane(vi, 0), t1 = __builtin_amdgcn_readlane(vi, 16);
    int t2 = __builtin_amdgcn_readlane(vi, 32), t3 = __builtin_amdgcn_readlane(vi, 48);
    __builtin_memcpy(&r0, &t0, 4);
    __builtin_memcpy(&r1, &t1, 4);
    __builtin_memcpy(&r2, &t2, 4);
    __builtin_memcpy(&r3, &t3, 4);
    return (r0 + r1) + (r2 + r3);
}

// Two workgroups (eight waves a SIMD) must fit: that caps the scalar
// registers the unrolled anchor loop may hoist.
template <bool BWD, bool INT_MODE, int NCMAX>
__global__ __launch_bounds__(kTbThreads) __attribute__((amdgpu_waves_per_eu(8))) void k_prod_pairs_tbl(
    const float *__restrict__ x1, const float *__restrict__ x2, const float *__restrict__ pe,
    const int2 *__restrict__ anchors, const double *__restrict__ P, float *__restrict__ cnt,
    float *__restrict__ x1_grad, float *__restrict__ x2_grad, float *__restrict__ pe_grad,
    uint32_t S, uint32_t n1, uint32_t n2, uint32_t pd, uint32_t T, uint32_t n_anchors, bool sliced,
    float cmp_eps, double int_rescaler, uint32_t JB, uint32_t n_jblocks) {
    // int32 payloads are summed as uint32 (wrapping, as the reference's int sums)
    typedef typename std::conditional<INT_MODE, uint32_t, float>::type push_t;
    // and the workgroup's sums of fp32 pushes are fp64
    typedef typename std::conditional<INT_MODE, uint32_t, double>::type acc_t;
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t E = 1u << n_anchors;
    const uint32_t NS = 2 * n_anchors;
    int2 *code = reinterpret_cast<int2 *>(smem);
    uint32_t *hist = reinterpret_cast<uint32_t *>(code + n_anchors);
    const uint32_t hist_words = (JB * E + 1) / 2;
    float *xs = reinterpret_cast<float *>(hist + ((hist_words + 1) & ~1u));  // 8-byte aligned
    const uint32_t tid = threadIdx.x;
    const uint32_t jblk = blockIdx.x % n_jblocks;
    const uint32_t bt = blockIdx.x / n_jblocks;
    const uint32_t t = bt % T, b = bt / T;
    const uint32_t j0 = jblk * JB;
    const uint32_t j_end = min(S, j0 + JB);
    const uint32_t R = j_end;  // rows 0 .. j_end-1 (i, j and distances all below j_end)
    acc_t *acc = reinterpret_cast<acc_t *>(xs + (size_t)R * NS);  // BWD only (NS is even)
    if (tid < n_anchors) {
        const int2 ap = anchors[(size_t)t * n_anchors + tid];
        int2 c = make_int2(-1, -1);
        int32_t s1, s2;
        uint32_t k1, k2;
        if (ap.x >= 0 && ap.y >= 0 && prod_locate(n1, n2, pd, sliced, (uint32_t)ap.x, s1, k1) &&
            prod_locate(n1, n2, pd, sliced, (uint32_t)ap.y, s2, k2))
            c = make_int2((s1 << 28) | (int32_t)(2 * tid * R), (s2 << 28) | (int32_t)((2 * tid + 1) * R));
        code[tid] = c;
    }
    for (uint32_t e = tid; e < hist_words; e += kTbThreads) hist[e] = 0;
    __syncthreads();
    // stage the slot values of rows 0 .. R-1 (positional slots: distance r, valid r < S-1)
    for (uint32_t e = tid; e < R * NS; e += kTbThreads) {
        const uint32_t sidx = e / R, r = e - sidx * R;
        const int2 c = code[sidx / 2];
        float v = 0.0f;
        if (c.x != -1) {
            const int2 ap = anchors[(size_t)t * n_anchors + sidx / 2];
            int32_t src;
            uint32_t k;
            prod_locate(n1, n2, pd, sliced, (uint32_t)((sidx & 1) ? ap.y : ap.x), src, k);
            if (src == 0) v = x1[((size_t)b * S + r) * n1 + k];
            else if (src == 1) v = x2[((size_t)b * S + r) * n2 + k];
            else if (r + 1 < S) v = pe[((size_t)r * T + t) * pd + k];
        }
        xs[e] = v;
        if (BWD) acc[e] = 0;
    }
    __syncthreads();
    const double *Pt = BWD ? P + (size_t)t * E : nullptr;
    const size_t TE = (size_t)T * E;
    const uint32_t lane = tid & 63;
    // the anchor codes are the same for every lane: scalar registers
    int32_t ca[NCMAX], cb[NCMAX];
#pragma unroll
    for (int a = 0; a < NCMAX; a++) {
        const int2 c = (uint32_t)a < n_anchors ? code[a] : make_int2(-1, -1);
        ca[a] = __builtin_amdgcn_readfirstlane(c.x);
        cb[a] = __builtin_amdgcn_readfirstlane(c.y);
    }
    const bool eps0 = cmp_eps == 0.0f;
    // pairs (i < j, j in the block), j-major, kTbThreads apart per thread
    uint32_t j = j0, i = tid;
    while (j < j_end && i >= j) {
        i -= j;
        j++;
    }
    while (true) {
        const bool active = j < j_end;
        const uint64_t act = __ballot(active);
        if (act == 0) break;  // wave-uniform: every lane of the wave leaves together
        // pushes into the shared row j, summed over the wave below
        int32_t ps0 = -1, ps1 = -1;
        push_t pv0 = 0, pv1 = 0;
        if (active) {
            const int32_t B0 = (int32_t)i, B1 = (int32_t)j, B2 = (int32_t)(j - i - 1);
            // every operand read is issued before the first compare
            float v1[NCMAX], v2[NCMAX];
#pragma unroll
            for (int a = 0; a < NCMAX; a++) {
                if (ca[a] == -1) continue;  // uniform
                const int32_t s1 = ca[a] >> 28, s2 = cb[a] >> 28;
                v1[a] = xs[(s1 == 0 ? B0 : (s1 == 1 ? B1 : B2)) + (ca[a] & 0xFFFFFFF)];
                v2[a] = xs[(s2 == 0 ? B0 : (s2 == 1 ? B1 : B2)) + (cb[a] & 0xFFFFFFF)];
            }
            int32_t idx = 0, flip = -1;
            float md = 3.402823466e+38f;
#pragma unroll
            for (int a = 0; a < NCMAX; a++) {
                if (ca[a] == -1) continue;
                const float dv = v1[a] - v2[a];
                // ROUNDED_COMPARISON_GREATER(dv, 0, cmp_eps), misc.h:16
                const bool gt = (dv > 0.0f) & (eps0 | !(fabsf(dv) < cmp_eps));
                idx |= gt ? (1 << a) : 0;
                if (fabsf(dv) < fabsf(md)) {
                    md = dv;
                    flip = a;
                }
            }
            const uint32_t h = (j - j0) * E + (uint32_t)idx;
            atomicAdd(&hist[h >> 1], 1u << (16 * (h & 1)));
            if (BWD && flip >= 0) {
                const double *Pbj = Pt + ((size_t)b * S + j) * TE;
                const double du = du_of_margin(md) * (Pbj[idx] - Pbj[idx ^ (1 << flip)]);
                if (fabs(du) > kEps) {
                    const int2 c = code[flip];
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const int32_t cc = hh == 0 ? c.x : c.y;
                        const int32_t sr = cc >> 28;
                        const double v = hh == 0 ? du : -du;
                        push_t pv;
                        if (INT_MODE) pv = (push_t)(uint32_t)(int32_t)(v * kDenom32 * int_rescaler);
                        else pv = (push_t)(float)v;
                        if (sr == 1) {
                            if (hh == 0) { ps0 = cc & 0xFFFFFFF; pv0 = pv; }
                            else { ps1 = cc & 0xFFFFFFF; pv1 = pv; }
                        } else {
                            atomicAdd(acc + (sr == 0 ? B0 : B2) + (cc & 0xFFFFFFF), (acc_t)pv);
                        }
                    }
                }
            }
        }
        if (BWD) {
            // every lane of the wave is here; the row j of the first active lane
            const uint32_t first = (uint32_t)__builtin_ctzll(act);
            const uint32_t jw = (uint32_t)__builtin_amdgcn_readlane((int)j, (int)first);
            const bool uniform = __ballot(active && j != jw) == 0;
            if (!uniform) {
                if (ps0 >= 0) atomicAdd(acc + ps0 + j, (acc_t)pv0);
                if (ps1 >= 0) atomicAdd(acc + ps1 + j, (acc_t)pv1);
            } else if (__ballot(ps0 >= 0 || ps1 >= 0) != 0) {
#pragma unroll
                for (int a = 0; a < NCMAX; a++) {
#pragma unroll
                    for (int hh = 0; hh < 2; hh++) {
                        const int32_t cc = hh == 0 ? ca[a] : cb[a];
                        if (cc == -1 || (cc >> 28) != 1) continue;  // uniform
                        const int32_t sb = cc & 0xFFFFFFF;
                        const push_t mine = (ps0 == sb ? pv0 : (push_t)0) + (ps1 == sb ? pv1 : (push_t)0);
                        if (__ballot(mine != (push_t)0) == 0) continue;
                        const push_t tot = wave_sum64(mine);
                        if (lane == first) atomicAdd(acc + sb + jw, (acc_t)tot);
                    }
                }
            }
        }
        if (active) {
            i += kTbThreads;
            while (j < j_end && i >= j) {
                i -= j;
                j++;
            }
        }
    }
    __syncthreads();
    for (uint32_t e = tid; e < (j_end - j0) * E; e += kTbThreads) {
        const uint32_t jj = e / E, ee = e - jj * E;
        cnt[((size_t)b * S + j0 + jj) * TE + (size_t)t * E + ee] = (float)((hist[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
    }
    if (BWD) {
        for (uint32_t e = tid; e < R * NS; e += kTbThreads) {
            const uint32_t sidx = e / R, r = e - sidx * R;
            const acc_t av = acc[e];
            if (av == (acc_t)0) continue;  // a zero sum (of either sign) adds nothing
            const int2 ap = anchors[(size_t)t * n_anchors + sidx / 2];
            int32_t src;
            uint32_t k;
            prod_locate(n1, n2, pd, sliced, (uint32_t)((sidx & 1) ? ap.y : ap.x), src, k);
            float *dst = src == 0 ? x1_grad + ((size_t)b * S + r) * n1 + k
                                  : (src == 1 ? x2_grad + ((size_t)b * S + r) * n2 + k
                                              : pe_grad + ((size_t)r * T + t) * pd + k);
            if (INT_MODE) atomicAdd(reinterpret_cast<int32_t *>(dst), (int32_t)av);
            else atomicAdd(dst, (float)av);
        }
    }
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

// The fp64 products on the matrix cores (v_mfma_f64_16x16x4f64).  A
// workgroup of WM x WN waves owns a (WM*WTM*16) x (WN*WTN*16) tile, each wave
// WTM x WTN MFMA tiles of 16 x 16; K runs in steps of 16 through a double
// buffer in LDS, fp64 (operands converted and, for BMODE 2, cut and scaled on
// the way in, exactly as the VALU kernel does), with the next step's global
// loads in flight while the current one multiplies.  Lane layout of the
// instruction (measured on gfx950): A[i][k] in lane i + 16k, B[k][j] in lane
// j + 16k, D[q + 4r][j] in register r of lane j + 16q -- not the fp32
// instruction's D[4q + r][j].  gridDim.z splits K; with a split the workgroup
// stores its fp64 partial tile to part[z] and k_prod_splitk_reduce adds the
// partials in z order (deterministic) into C.
typedef double f64x4 __attribute__((ext_vector_type(4)));
constexpr int kMfK = 16;

template <int WTM, int WTN, int WM, int WN, bool TA, bool TB, int BMODE, int OUT>
__global__ __launch_bounds__(64 * WM * WN) void k_prod_gemm_mfma(
    const float *__restrict__ A, uint32_t lda, const float *__restrict__ B, uint32_t ldb,
    void *__restrict__ C, double *__restrict__ part, uint32_t M, uint32_t N, uint32_t K,
    uint32_t k_chunk, double lr) {
    constexpr int TM = WM * WTM * 16, TN = WN * WTN * 16, NT = 64 * WM * WN;
    constexpr int LA = TM * kMfK / NT, LB = kMfK * TN / NT;
    static_assert(LA * NT == TM * kMfK && LB * NT == kMfK * TN, "tile does not split over threads");
    __shared__ double As[2][kMfK][TM + 1];
    __shared__ double Bs[2][kMfK][TN + 1];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t wm = (wave % WM) * WTM * 16, wn = (wave / WM) * WTN * 16;
    const uint32_t li = lane & 15, lq = lane >> 4;
    const uint32_t m0 = blockIdx.y * TM, n0 = blockIdx.x * TN;
    const uint32_t kb = blockIdx.z * k_chunk, ke = min(K, kb + k_chunk);
    f64x4 acc[WTM][WTN];
#pragma unroll
    for (int a = 0; a < WTM; a++)
#pragma unroll
        for (int b = 0; b < WTN; b++) acc[a][b] = f64x4{0.0, 0.0, 0.0, 0.0};
    float ra[LA], rb[LB];
    // element e of a tile: the index order follows the source's contiguous
    // dimension, for coalescing
    auto gload = [&](uint32_t k0) {
#pragma unroll
        for (int u = 0; u < LA; u++) {
            const uint32_t e = tid + NT * u;
            const uint32_t mm = TA ? e % TM : e / kMfK, kk = TA ? e / TM : e % kMfK;
            const uint32_t m = m0 + mm, k = k0 + kk;
            ra[u] = (m < M && k < ke) ? (TA ? A[(size_t)k * lda + m] : A[(size_t)m * lda + k]) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < LB; u++) {
            const uint32_t e = tid + NT * u;
            const uint32_t nn = TB ? e / kMfK : e % TN, kk = TB ? e % kMfK : e / TN;
            const uint32_t n = n0 + nn, k = k0 + kk;
            rb[u] = (n < N && k < ke) ? (TB ? B[(size_t)n * ldb + k] : B[(size_t)k * ldb + n]) : 0.0f;
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int u = 0; u < LA; u++) {
            const uint32_t e = tid + NT * u;
            const uint32_t mm = TA ? e % TM : e / kMfK, kk = TA ? e / TM : e % kMfK;
            As[buf][kk][mm] = (double)ra[u];
        }
#pragma unroll
        for (int u = 0; u < LB; u++) {
            const uint32_t e = tid + NT * u;
            const uint32_t nn = TB ? e / kMfK : e % TN, kk = TB ? e % kMfK : e / TN;
            double bt = (double)rb[u];
            if (BMODE == 2) bt = (fabs(bt) > kEps) ? bt * lr : 0.0;
            Bs[buf][kk][nn] = bt;
        }
    };
    int buf = 0;
    if (kb < ke) {
        gload(kb);
        lstore(0);
    }
    __syncthreads();
    for (uint32_t k0 = kb; k0 < ke; k0 += kMfK) {
        const bool more = k0 + kMfK < ke;
        if (more) gload(k0 + kMfK);
#pragma unroll
        for (int ks = 0; ks < kMfK / 4; ks++) {
            const uint32_t kr = ks * 4 + lq;
            double av[WTM], bv[WTN];
#pragma unroll
            for (int a = 0; a < WTM; a++) av[a] = As[buf][kr][wm + a * 16 + li];
#pragma unroll
            for (int b = 0; b < WTN; b++) bv[b] = Bs[buf][kr][wn + b * 16 + li];
#pragma unroll
            for (int a = 0; a < WTM; a++)
#pragma unroll
                for (int b = 0; b < WTN; b++)
                    acc[a][b] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
        if (more) lstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    double *pz = part ? part + (size_t)blockIdx.z * M * N : nullptr;
#pragma unroll
    for (int a = 0; a < WTM; a++)
#pragma unroll
        for (int b = 0; b < WTN; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t m = m0 + wm + a * 16 + lq + 4 * r;
                const uint32_t n = n0 + wn + b * 16 + li;
                if (m >= M || n >= N) continue;
                const size_t o = (size_t)m * N + n;
                const double v = acc[a][b][r];
                if (pz) {
                    pz[o] = v;
                } else if (OUT == 0) {
                    float *Cf = reinterpret_cast<float *>(C);
                    Cf[o] = (float)((double)Cf[o] + v);
                } else {
                    reinterpret_cast<double *>(C)[o] = v;
                }
            }
}

template <int OUT>
__global__ __launch_bounds__(256) void k_prod_splitk_reduce(const double *__restrict__ part,
                                                            void *__restrict__ C, uint64_t MN,
                                                            uint32_t splits) {
    for (uint64_t o = (uint64_t)blockIdx.x * 256 + threadIdx.x; o < MN; o += (uint64_t)gridDim.x * 256) {
        double v = 0.0;
        for (uint32_t z = 0; z < splits; z++) v += part[(size_t)z * MN + o];
        if (OUT == 0) {
            float *Cf = reinterpret_cast<float *>(C);
            Cf[o] = (float)((double)Cf[o] + v);
        } else {
            reinterpret_cast<double *>(C)[o] = v;
        }
    }
}

// K splits of the 64 x 64-tile products: about 2048 workgroups (eight per
// CU), each split at least 256 deep.
uint32_t splitk_for(uint32_t M, uint32_t N, uint32_t K) {
    const uint64_t tiles = (uint64_t)((M + 63) / 64) * ((N + 63) / 64);
    uint64_t split = (2048 + tiles - 1) / tiles;
    const uint64_t max_split = K / 256 > 0 ? K / 256 : 1;
    if (split > max_split) split = max_split;
    if (split > 16) split = 16;
    return (uint32_t)(split < 1 ? 1 : split);
}

size_t splitk_bytes(uint32_t M, uint32_t N, uint32_t K) {
    const uint32_t z = splitk_for(M, N, K);
    return z > 1 ? (size_t)z * M * N * 8 : 0;
}

// part == nullptr: one pass over K on the 128 x 64 tile (the product whose
// output tiles already fill the chip); else the 64 x 64 tile split over K.
template <bool TA, bool TB, int BMODE, int OUT>
hipError_t gemm_mfma(const float *A, uint32_t lda, const float *B, uint32_t ldb, void *C, uint32_t M,
                     uint32_t N, uint32_t K, double lr, double *part, hipStream_t st) {
    if (M == 0 || N == 0) return hipSuccess;
    if (!part) {
        const dim3 grid((N + 63) / 64, (M + 127) / 128, 1);
        if (grid.y > 65535u) return hipErrorInvalidConfiguration;
        hipLaunchKernelGGL((k_prod_gemm_mfma<4, 2, 2, 2, TA, TB, BMODE, OUT>), grid, dim3(256), 0, st,
                           A, lda, B, ldb, C, (double *)nullptr, M, N, K, K, lr);
        return hipGetLastError();
    }
    const uint32_t z = splitk_for(M, N, K);
    const uint32_t k_chunk = ((K + z - 1) / z + kMfK - 1) / kMfK * kMfK;
    const dim3 grid((N + 63) / 64, (M + 63) / 64, z);
    if (grid.y > 65535u) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((k_prod_gemm_mfma<2, 2, 2, 2, TA, TB, BMODE, OUT>), grid, dim3(256), 0, st, A,
                       lda, B, ldb, C, z > 1 ? part : nullptr, M, N, K, k_chunk, lr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || z == 1) return e;
    const uint64_t MN = (uint64_t)M * N;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((MN + 255) / 256, 4096);
    hipLaunchKernelGGL((k_prod_splitk_reduce<OUT>), dim3(blocks), dim3(256), 0, st, part, C, MN, z);
    return hipGetLastError();
}

// Product mode over sparse lookup connectivity (this build's CSR, weights per
// synapse): one thread per (b, table, pair), the reference's own
// decomposition with fp32 / int32 atomics (fill_outputs_product_sparse_logic,
// proto:2266-2394; propagate_backward_product_cpu_logic, proto:2396-2628: the
// main and flipped sums over every synapse of the two neurons, one du per
// pair; gather_w_gradients_product_sparse, proto:2946-3073: every synapse of
// the pair's neuron).  MODE 0: forward; 1: input / positional gradients, and
// the weight gradient when target is given; 2: the weight gradient alone (the
// Internal policy, after mode 1 read the weights).
template <int MODE, bool INT_MODE>
__global__ __launch_bounds__(256) void k_prod_sparse(
    const float *__restrict__ x1, const float *__restrict__ x2, const float *__restrict__ pe,
    const int2 *__restrict__ anchors, const float *__restrict__ w, const int64_t *__restrict__ off,
    const int32_t *__restrict__ tgt, const float *__restrict__ g, float *__restrict__ out,
    float *__restrict__ x1_grad, float *__restrict__ x2_grad, float *__restrict__ pe_grad,
    float *__restrict__ target, uint32_t S, uint32_t n1, uint32_t n2, uint32_t pd, uint32_t T,
    uint32_t n_anchors, uint32_t O, bool sliced, float cmp_eps, double lr, double int_rescaler,
    uint64_t n_pairs, uint64_t n_items) {
    const uint64_t item = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (item >= n_items) return;
    const uint64_t p = item % n_pairs;
    const uint64_t bt = item / n_pairs;
    const uint32_t t = (uint32_t)(bt % T), b = (uint32_t)(bt / T);
    uint64_t jj = (uint64_t)((1.0 + sqrt(1.0 + 8.0 * (double)p)) * 0.5);
    while (jj * (jj - 1) / 2 > p) jj--;
    while ((jj + 1) * jj / 2 <= p) jj++;
    const uint32_t j = (uint32_t)jj, i = (uint32_t)(p - jj * (jj - 1) / 2);
    const size_t pe_off = ((size_t)(j - i - 1) * T + t) * pd;
    const PairLookup lk = prod_lookup(x1 + ((size_t)b * S + i) * n1, x2 + ((size_t)b * S + j) * n2,
                                      pd ? pe + pe_off : nullptr, anchors + (size_t)t * n_anchors,
                                      n_anchors, n1, n2, pd, sliced, cmp_eps);
    const uint32_t n = t * (1u << n_anchors) + (uint32_t)lk.idx;
    const size_t orow = ((size_t)b * S + j) * O;
    if (MODE == 0) {
        for (int64_t sy = off[n]; sy < off[n + 1]; sy++) {
            const uint32_t o = (uint32_t)tgt[sy];
            if (o >= O) continue;
            if (INT_MODE) atomicAdd(reinterpret_cast<int32_t *>(out + orow + o), (int32_t)((double)w[sy] * kDenom32 * int_rescaler));
            else unsafeAtomicAdd(out + orow + o, w[sy]);
        }
        return;
    }
    const float *gj = g + orow;
    if (MODE == 1 && lk.src1 >= 0) {
        const uint32_t na = t * (1u << n_anchors) + (uint32_t)lk.alt;
        double ms = 0.0, as = 0.0;
        for (int64_t sy = off[n]; sy < off[n + 1]; sy++) {
            const uint32_t o = (uint32_t)tgt[sy];
            if (o < O) ms += (double)w[sy] * (double)gj[o];
        }
        for (int64_t sy = off[na]; sy < off[na + 1]; sy++) {
            const uint32_t o = (uint32_t)tgt[sy];
            if (o < O) as += (double)w[sy] * (double)gj[o];
        }
        const double du = du_of_margin(lk.md) * (ms - as);
        if (fabs(du) > kEps) {
            float *dst[3] = {x1_grad + ((size_t)b * S + i) * n1, x2_grad + ((size_t)b * S + j) * n2,
                             pd ? pe_grad + pe_off : nullptr};
            const int32_t srcs[2] = {lk.src1, lk.src2};
            const uint32_t ks[2] = {lk.k1, lk.k2};
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float *d = dst[srcs[h]];
                if (!d) continue;
                const double v = h == 0 ? du : -du;
                if (INT_MODE) atomicAdd(reinterpret_cast<int32_t *>(d + ks[h]), (int32_t)(v * kDenom32 * int_rescaler));
                else unsafeAtomicAdd(d + ks[h], (float)v);
            }
        }
    }
    if (target) {
        for (int64_t sy = off[n]; sy < off[n + 1]; sy++) {
            const uint32_t o = (uint32_t)tgt[sy];
            if (o >= O) continue;
            const double gg = (double)gj[o];
            if (!(fabs(gg) > kEps)) continue;
            if (INT_MODE) atomicAdd(reinterpret_cast<int32_t *>(target + sy), (int32_t)(gg * lr * kDenom32 * int_rescaler));
            else unsafeAtomicAdd(target + sy, (float)(gg * lr));
        }
    }
}

template <int MODE, bool IM>
hipError_t launch_prod_sparse(const ProductShape &s, const float *x1, const float *x2, const float *pe,
                              const int32_t *anchors, const float *w, const int64_t *off,
                              const int32_t *tgt, const float *g, float *out, float *x1_grad,
                              float *x2_grad, float *pe_grad, float *target, double lr,
                              double int_rescaler, hipStream_t st) {
    const uint64_t n_pairs = (uint64_t)s.seq_len * (s.seq_len - 1) / 2;
    const uint64_t n_items = (uint64_t)s.batch * s.n_detectors * n_pairs;
    if (n_items == 0) return hipSuccess;
    const uint64_t blocks = (n_items + 255) / 256;
    if (blocks > 0x7fffffffull) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((k_prod_sparse<MODE, IM>), dim3((uint32_t)blocks), dim3(256), 0, st, x1, x2, pe,
                       reinterpret_cast<const int2 *>(anchors), w, off, tgt, g, out, x1_grad, x2_grad,
                       pe_grad, target, s.seq_len, s.n1, s.n2, s.pd, s.n_detectors, s.n_anchors,
                       s.n_outputs, s.sliced, s.cmp_eps, lr, int_rescaler, n_pairs, n_items);
    return hipGetLastError();
}

}  // namespace

bool product_applies(const ProductShape &s) {
    const uint64_t TE = (uint64_t)s.n_detectors << s.n_anchors;
    return s.n_anchors <= 16 && TE <= kPrMaxHist && (uint64_t)s.batch * s.seq_len <= 0x7fffffffu &&
           (uint64_t)s.batch * s.seq_len <= 65535ull * kGmTile;
}

// scratch: Cnt [B*S][T*E] f32 | P [B*S][T*E] f64 (backward) | split-K partials
// of the product that sums over the longest dimension (forward: Cnt . W over
// T*E; backward: Cnt^T . g' over B*S)

hipError_t launch_forward_product(const ProductShape &s, const float *w, const float *x1,
                                  const float *x2, const float *pe, const int32_t *anchors,
                                  float *out, bool int_mode, double int_rescaler, Scratch &scratch,
                                  hipStream_t st) {
    const uint32_t E = 1u << s.n_anchors;
    const uint32_t TE = s.n_detectors * E;
    const uint32_t BS = s.batch * s.seq_len;
    ScratchLayout sl(scratch);
    float *cnt = sl.take<float>((size_t)BS * TE * 4);
    double *part = sl.take<double>(splitk_bytes(BS, s.n_outputs, TE));
    hipError_t e;
    if (sl.stop(&e, "forward_step_product")) return e;
    if (BS == 0) return hipSuccess;
    const int2 *anc = reinterpret_cast<const int2 *>(anchors);
    const TableLayout lay = table_grid_ok(s, table_layout(s, false, 0));
    const uint32_t njb = lay.jb ? (s.seq_len + lay.jb - 1) / lay.jb : 0;
#define SPIKY_PT(IM, NCM)                                                                         \
    hipLaunchKernelGGL((k_prod_pairs_tbl<false, IM, NCM>), dim3(s.batch * s.n_detectors * njb),   \
                       dim3(kTbThreads), lay.bytes, st, x1, x2, pe, anc, (const double *)nullptr, \
                       cnt, (float *)nullptr, (float *)nullptr, (float *)nullptr, s.seq_len,      \
                       s.n1, s.n2, s.pd, s.n_detectors, s.n_anchors, s.sliced, s.cmp_eps,         \
                       int_rescaler, lay.jb, njb)
#define SPIKY_PP(IM)                                                                              \
    if (lay.jb) {                                                                                 \
        if (s.n_anchors <= 4) SPIKY_PT(IM, 4);                                                    \
        else if (s.n_anchors <= 8) SPIKY_PT(IM, 8);                                               \
        else SPIKY_PT(IM, 16);                                                                    \
    } else                                                                                        \
        hipLaunchKernelGGL((k_prod_pairs<false, IM>), dim3(BS), dim3(kPrThreads), TE * 4, st, x1, \
                           x2, pe, anc, (const double *)nullptr, cnt, (float *)nullptr,           \
                           (float *)nullptr, (float *)nullptr, s.seq_len, s.n1, s.n2, s.pd,       \
                           s.n_detectors, s.n_anchors, s.sliced, s.cmp_eps, int_rescaler)
    if (int_mode) { SPIKY_PP(true); } else { SPIKY_PP(false); }
#undef SPIKY_PP
#undef SPIKY_PT
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // out[bj][o] (+)= sum_k cnt[bj][k] * W[k][o]
    if (int_mode)
        return gemm<false, false, 1, 1>(cnt, TE, w, s.n_outputs, out, BS, s.n_outputs, TE, 0.0,
                                        int_rescaler, st);
    return gemm_mfma<false, false, 0, 0>(cnt, TE, w, s.n_outputs, out, BS, s.n_outputs, TE, 0.0, part,
                                         st);
}

hipError_t launch_backward_product(const ProductShape &s, const float *w, const float *x1,
                                   const float *x2, const float *pe, const int32_t *anchors,
                                   const float *g, float *x1_grad, float *x2_grad, float *pe_grad,
                                   float *target, double lr, bool int_mode, double int_rescaler,
                                   Scratch &scratch, hipStream_t st) {
    const uint32_t E = 1u << s.n_anchors;
    const uint32_t TE = s.n_detectors * E;
    const uint32_t BS = s.batch * s.seq_len;
    ScratchLayout sl(scratch);
    float *cnt = sl.take<float>((size_t)BS * TE * 4);
    double *P = sl.take<double>((size_t)BS * TE * 8);
    double *part = sl.take<double>(splitk_bytes(TE, s.n_outputs, BS));
    hipError_t e;
    if (sl.stop(&e, "backward_backprop_product")) return e;
    if (BS == 0) return hipSuccess;
    // P[bj][k] = sum_o g[bj][o] * W[k][o]  (fp64; no split: B*S x T*E tiles fill the chip)
    e = gemm_mfma<false, true, 0, 2>(g, s.n_outputs, w, s.n_outputs, P, BS, TE,
                                                s.n_outputs, 0.0, nullptr, st);
    if (e != hipSuccess) return e;
    const int2 *anc = reinterpret_cast<const int2 *>(anchors);
    const TableLayout lay = table_grid_ok(s, table_layout(s, true, int_mode ? 4 : 8));
    const uint32_t njb = lay.jb ? (s.seq_len + lay.jb - 1) / lay.jb : 0;
#define SPIKY_BT(IM, NCM)                                                                         \
    hipLaunchKernelGGL((k_prod_pairs_tbl<true, IM, NCM>), dim3(s.batch * s.n_detectors * njb),    \
                       dim3(kTbThreads), lay.bytes, st, x1, x2, pe, anc, P, cnt, x1_grad,         \
                       x2_grad, pe_grad, s.seq_len, s.n1, s.n2, s.pd, s.n_detectors, s.n_anchors, \
                       s.sliced, s.cmp_eps, int_rescaler, lay.jb, njb)
#define SPIKY_PB(IM)                                                                              \
    if (lay.jb) {                                                                                 \
        if (s.n_anchors <= 4) SPIKY_BT(IM, 4);                                                    \
        else if (s.n_anchors <= 8) SPIKY_BT(IM, 8);                                               \
        else SPIKY_BT(IM, 16);                                                                    \
    } else                                                                                        \
        hipLaunchKernelGGL((k_prod_pairs<true, IM>), dim3(BS), dim3(kPrThreads), TE * 4, st, x1,  \
                           x2, pe, anc, P, cnt, x1_grad, x2_grad, pe_grad, s.seq_len, s.n1, s.n2, \
                           s.pd, s.n_detectors, s.n_anchors, s.sliced, s.cmp_eps, int_rescaler)
    if (int_mode) { SPIKY_PB(true); } else { SPIKY_PB(false); }
#undef SPIKY_PB
#undef SPIKY_BT
    e = hipGetLastError();
    if (e != hipSuccess || target == nullptr) return e;
    // target[k][o] (+)= sum_bj cnt[bj][k] * g'[bj][o]
    if (int_mode)
        return gemm<true, false, 2, 1>(cnt, TE, g, s.n_outputs, target, TE, s.n_outputs, BS, lr,
                                       int_rescaler, st);
    return gemm_mfma<true, false, 2, 0>(cnt, TE, g, s.n_outputs, target, TE, s.n_outputs, BS, lr,
                                        part, st);
}

}  // namespace spiky

namespace spiky {

bool product_sparse_applies(const ProductShape &s) {
    const uint64_t n_items = (uint64_t)s.batch * s.n_detectors * ((uint64_t)s.seq_len * (s.seq_len - 1) / 2);
    return s.n_anchors <= 24 && (n_items + 255) / 256 <= 0x7fffffffull;
}

hipError_t launch_forward_product_sparse(const ProductShape &s, const float *w, const float *x1,
                                         const float *x2, const float *pe, const int32_t *anchors,
                                         const int64_t *syn_offsets, const int32_t *syn_targets,
                                         float *out, bool int_mode, double int_rescaler,
                                         hipStream_t st) {
    if (int_mode)
        return launch_prod_sparse<0, true>(s, x1, x2, pe, anchors, w, syn_offsets, syn_targets, nullptr,
                                           out, nullptr, nullptr, nullptr, nullptr, 0.0, int_rescaler, st);
    return launch_prod_sparse<0, false>(s, x1, x2, pe, anchors, w, syn_offsets, syn_targets, nullptr, out,
                                        nullptr, nullptr, nullptr, nullptr, 0.0, int_rescaler, st);
}

hipError_t launch_backward_product_sparse(const ProductShape &s, const float *w, const float *x1,
                                          const float *x2, const float *pe, const int32_t *anchors,
                                          const int64_t *syn_offsets, const int32_t *syn_targets,
                                          const float *g, float *x1_grad, float *x2_grad,
                                          float *pe_grad, float *target, double lr, bool int_mode,
                                          double int_rescaler, hipStream_t st) {
    // the Internal policy updates the weights: after the input gradient read them
    const bool internal = target == w;
    float *t1 = internal ? nullptr : target;
    hipError_t e = int_mode
        ? launch_prod_sparse<1, true>(s, x1, x2, pe, anchors, w, syn_offsets, syn_targets, g, nullptr,
                                      x1_grad, x2_grad, pe_grad, t1, lr, int_rescaler, st)
        : launch_prod_sparse<1, false>(s, x1, x2, pe, anchors, w, syn_offsets, syn_targets, g, nullptr,
                                       x1_grad, x2_grad, pe_grad, t1, lr, int_rescaler, st);
    if (e != hipSuccess || !internal) return e;
    return int_mode ? launch_prod_sparse<2, true>(s, x1, x2, pe, anchors, w, syn_offsets, syn_targets, g,
                                                  nullptr, nullptr, nullptr, nullptr, target, lr,
                                                  int_rescaler, st)
                    : launch_prod_sparse<2, false>(s, x1, x2, pe, anchors, w, syn_offsets, syn_targets, g,
                                                   nullptr, nullptr, nullptr, nullptr, target, lr,
                                                   int_rescaler, st);
}

}  // namespace spiky
