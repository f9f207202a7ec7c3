// lut_seq_sparse.hip -- sequence-concat mode over sparse lookup connectivity
// (a Conv2DLUTLayer attention with a lookup receptive field), gfx950.
//
// Connectivity is this build's CSR (lut_kernels.h): lookup neuron n owns
// synapses [syn_offsets[n], syn_offsets[n+1]) with output indices
// syn_targets[s] and one weight w[s] each; forward group g of a neuron is its
// synapses g*fgs .. g*fgs+fgs-1 in list order.  Every causal pair (i < j) of
// a sequence and table t looks up neuron
//   n = t * 2^(2Nc+Npe) + (Q_j << (Nc+Npe) | K_i << Npe | PE_(j-i-1)),
// as the reference's fill_outputs_sparse_seq_logic (lut_runtime_kernels_logic.
// proto:1906-2015), propagate_through_detectors_seq_sparse_logic
// (proto:3371-3627) and gather_w_gradients_seq_sparse_logic (proto:3837-3942).
//
// One thread per (b, group, table, pair), the reference's own decomposition,
// with fp32 / int32 atomics: this path serves topologies without a benchmark
// configuration, so it is built for parity, not speed.  int32 payload sums are
// order-free and bit-exact; fp32 sums hold the reference's terms in another
// order.
#include "lut_kernels.h"

namespace spiky {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ double du_of_margin(float md) {
    double du = (double)md;
    double r = 1.0 / (1.0 + fabs(du));
    return (du > 0) ? r * (0.5 * r) : r * (-0.5 * r);
}

struct SeqSparseArgs {
    uint32_t batch, seq, n_inputs, n_outputs, n_detectors, n_anchors, pe_dim, fgs, max_groups;
    uint64_t n_pairs;  // S(S-1)/2
};

// item -> (b, group, t, i, j) with i < j; false past the end
__device__ __forceinline__ bool decode_item(const SeqSparseArgs &a, uint64_t item, uint32_t &b,
                                            uint32_t &grp, uint32_t &t, uint32_t &i, uint32_t &j) {
    const uint64_t n_items = (uint64_t)a.batch * a.max_groups * a.n_detectors * a.n_pairs;
    if (item >= n_items) return false;
    const uint64_t p = item % a.n_pairs;
    uint64_t rest = item / a.n_pairs;
    t = (uint32_t)(rest % a.n_detectors);
    rest /= a.n_detectors;
    grp = (uint32_t)(rest % a.max_groups);
    b = (uint32_t)(rest / a.max_groups);
    // pair p = j(j-1)/2 + i
    uint64_t jj = (uint64_t)((1.0 + sqrt(1.0 + 8.0 * (double)p)) * 0.5);
    while (jj * (jj - 1) / 2 > p) jj--;
    while ((jj + 1) * jj / 2 <= p) jj++;
    j = (uint32_t)jj;
    i = (uint32_t)(p - jj * (jj - 1) / 2);
    return true;
}

__device__ __forceinline__ uint32_t seq_neuron(uint32_t t, int32_t Q, int32_t K, int32_t P,
                                               uint32_t n_anchors, uint32_t pd) {
    const uint32_t row = ((uint32_t)Q << (n_anchors + pd)) | ((uint32_t)K << pd) | (uint32_t)P;
    return t * (1u << (2 * n_anchors + pd)) + row;
}

__device__ __forceinline__ void group_range(const int64_t *off, uint32_t n, uint32_t grp,
                                            uint32_t fgs, int64_t &s0, int64_t &s1) {
    s0 = off[n] + (int64_t)grp * fgs;
    s1 = min(s0 + (int64_t)fgs, off[n + 1]);
}

template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_fill_seq_sparse(
    SeqSparseArgs a, const float *__restrict__ w, const int32_t *__restrict__ idx,
    const int32_t *__restrict__ pidx, const int64_t *__restrict__ off,
    const int32_t *__restrict__ tgt, float *__restrict__ out, double int_rescaler) {
    uint32_t b, grp, t, i, j;
    if (!decode_item(a, (uint64_t)blockIdx.x * kBlock + threadIdx.x, b, grp, t, i, j)) return;
    const int32_t K = idx[((size_t)b * a.seq + i) * a.n_detectors + t];
    const int32_t Q = idx[((size_t)b * a.seq + j) * a.n_detectors + t];
    const int32_t P = a.pe_dim ? pidx[(size_t)(j - i - 1) * a.n_detectors + t] : 0;
    const uint32_t n = seq_neuron(t, Q, K, P, a.n_anchors, a.pe_dim);
    int64_t s0, s1;
    group_range(off, n, grp, a.fgs, s0, s1);
    float *oj = out + ((size_t)b * a.seq + j) * a.n_outputs;
    for (int64_t s = s0; s < s1; s++) {
        const uint32_t o = (uint32_t)tgt[s];
        if (o >= a.n_outputs) continue;
        const double wt = (double)w[s];
        if (INT_MODE) atomicAdd(reinterpret_cast<int32_t *>(oj + o), (int32_t)(wt * kDenom32 * int_rescaler));
        else unsafeAtomicAdd(oj + o, (float)wt);
    }
}

__device__ __forceinline__ double group_dot(const float *w, const int64_t *off, const int32_t *tgt,
                                            uint32_t n, uint32_t grp, uint32_t fgs, const float *gj,
                                            uint32_t n_outputs) {
    int64_t s0, s1;
    group_range(off, n, grp, fgs, s0, s1);
    double acc = 0.0;
    for (int64_t s = s0; s < s1; s++) {
        const uint32_t o = (uint32_t)tgt[s];
        if (o < n_outputs) acc += (double)w[s] * (double)gj[o];
    }
    return acc;
}

template <bool INT_MODE>
__device__ __forceinline__ void push(float *dst, double v, double int_rescaler) {
    if (INT_MODE) atomicAdd(reinterpret_cast<int32_t *>(dst), (int32_t)(v * kDenom32 * int_rescaler));
    else unsafeAtomicAdd(dst, (float)v);
}

template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_propagate_seq_sparse(
    SeqSparseArgs a, const float *__restrict__ w, const float *__restrict__ g,
    const int32_t *__restrict__ idx, const float *__restrict__ md, const int32_t *__restrict__ mi,
    const int32_t *__restrict__ pidx, const float *__restrict__ pmd, const int32_t *__restrict__ pmi,
    const int2 *__restrict__ anchors, const int64_t *__restrict__ off,
    const int32_t *__restrict__ tgt, float *__restrict__ x_grad, float *__restrict__ pe_grad,
    double int_rescaler) {
    uint32_t b, grp, t, i, j;
    if (!decode_item(a, (uint64_t)blockIdx.x * kBlock + threadIdx.x, b, grp, t, i, j)) return;
    const size_t ko = ((size_t)b * a.seq + i) * a.n_detectors + t;
    const size_t qo = ((size_t)b * a.seq + j) * a.n_detectors + t;
    const int32_t K = idx[ko], Q = idx[qo];
    const int32_t km = mi[ko], qm = mi[qo];
    const float kd = md[ko], qd = md[qo];
    const size_t pe_off = (size_t)(j - i - 1) * a.n_detectors + t;
    int32_t P = 0, pm = -1;
    float pdl = 0.0f;
    if (a.pe_dim) {
        P = pidx[pe_off];
        pm = pmi[pe_off];
        pdl = pmd[pe_off];
    }
    const float *gj = g + ((size_t)b * a.seq + j) * a.n_outputs;
    const uint32_t main_n = seq_neuron(t, Q, K, P, a.n_anchors, a.pe_dim);
    // flip Q's min anchor if |dQ| < |dK|, else K's (proto:3500-3530)
    const bool qflip = fabsf(qd) < fabsf(kd);
    const int32_t flip = qflip ? qm : km;
    const uint32_t alt_n = qflip ? seq_neuron(t, qm >= 0 ? Q ^ (1 << qm) : Q, K, P, a.n_anchors, a.pe_dim)
                                 : seq_neuron(t, Q, km >= 0 ? K ^ (1 << km) : K, P, a.n_anchors, a.pe_dim);
    const double ms = group_dot(w, off, tgt, main_n, grp, a.fgs, gj, a.n_outputs);
    const double as = group_dot(w, off, tgt, alt_n, grp, a.fgs, gj, a.n_outputs);
    const double du = du_of_margin(qflip ? qd : kd) * (ms - as);
    if (flip >= 0 && (uint32_t)flip < a.n_anchors && fabs(du) > kEps) {
        // propagate_through_detector, proto:821-867
        const int2 ap = anchors[(size_t)t * a.n_anchors + flip];
        const uint32_t pos = qflip ? j : i;
        float *xg = x_grad + ((size_t)b * a.seq + pos) * a.n_inputs;
        if ((uint32_t)ap.x < a.n_inputs && (uint32_t)ap.y < a.n_inputs) {
            push<INT_MODE>(xg + ap.x, du, int_rescaler);
            push<INT_MODE>(xg + ap.y, -du, int_rescaler);
        }
    }
    if (a.pe_dim && fabsf(pdl) < fabsf(qd) && fabsf(pdl) < fabsf(kd) && pm >= 0 &&
        (uint32_t)pm < a.pe_dim) {
        // update_positional_gradients, proto:1016-1046 (no EPS cut)
        const uint32_t pe_n = seq_neuron(t, Q, K, P ^ (1 << pm), a.n_anchors, a.pe_dim);
        const double dpe = du_of_margin(pdl) * (ms - group_dot(w, off, tgt, pe_n, grp, a.fgs, gj, a.n_outputs));
        push<INT_MODE>(pe_grad + pe_off * a.pe_dim + pm, dpe, int_rescaler);
    }
}

template <bool INT_MODE>
__global__ __launch_bounds__(kBlock) void k_wgrad_seq_sparse(
    SeqSparseArgs a, const float *__restrict__ g, const int32_t *__restrict__ idx,
    const int32_t *__restrict__ pidx, const int64_t *__restrict__ off,
    const int32_t *__restrict__ tgt, float *__restrict__ target, double lr, double int_rescaler) {
    uint32_t b, grp, t, i, j;
    if (!decode_item(a, (uint64_t)blockIdx.x * kBlock + threadIdx.x, b, grp, t, i, j)) return;
    const int32_t K = idx[((size_t)b * a.seq + i) * a.n_detectors + t];
    const int32_t Q = idx[((size_t)b * a.seq + j) * a.n_detectors + t];
    const int32_t P = a.pe_dim ? pidx[(size_t)(j - i - 1) * a.n_detectors + t] : 0;
    const uint32_t n = seq_neuron(t, Q, K, P, a.n_anchors, a.pe_dim);
    int64_t s0, s1;
    group_range(off, n, grp, a.fgs, s0, s1);
    const float *gj = g + ((size_t)b * a.seq + j) * a.n_outputs;
    for (int64_t s = s0; s < s1; s++) {
        const uint32_t o = (uint32_t)tgt[s];
        if (o >= a.n_outputs) continue;
        const double gg = (double)gj[o];
        if (!(fabs(gg) > kEps)) continue;
        // gather_weight_gradients_sparse, proto:584-714
        if (INT_MODE) atomicAdd(reinterpret_cast<int32_t *>(target + s), (int32_t)(gg * lr * kDenom32 * int_rescaler));
        else unsafeAtomicAdd(target + s, (float)(gg * lr));
    }
}

SeqSparseArgs make_args(const SeqShape &s, uint32_t max_groups) {
    SeqSparseArgs a;
    a.batch = s.batch;
    a.seq = s.seq;
    a.n_inputs = s.n_inputs;
    a.n_outputs = s.n_outputs;
    a.n_detectors = s.n_detectors;
    a.n_anchors = s.n_anchors;
    a.pe_dim = s.pe_dim;
    a.fgs = s.ogs;
    a.max_groups = max_groups;
    a.n_pairs = (uint64_t)s.seq * (s.seq - 1) / 2;
    return a;
}

bool grid_for(const SeqSparseArgs &a, uint32_t &blocks) {
    const uint64_t n = (uint64_t)a.batch * a.max_groups * a.n_detectors * a.n_pairs;
    const uint64_t bl = (n + kBlock - 1) / kBlock;
    if (bl > 0x7fffffffull) return false;
    blocks = (uint32_t)bl;
    return true;
}

}  // namespace

bool seq_sparse_applies(const SeqShape &s, uint32_t max_groups) {
    SeqSparseArgs a = make_args(s, max_groups);
    uint32_t blocks;
    return 2 * s.n_anchors + s.pe_dim <= 24 && grid_for(a, blocks);
}

hipError_t launch_fill_seq_sparse(const SeqShape &s, uint32_t max_groups, const float *w,
                                  const int32_t *idx, const int32_t *pidx, const int64_t *syn_offsets,
                                  const int32_t *syn_targets, float *out, bool int_mode,
                                  double int_rescaler, hipStream_t st) {
    const SeqSparseArgs a = make_args(s, max_groups);
    uint32_t blocks = 0;
    if (!grid_for(a, blocks)) return hipErrorInvalidConfiguration;
    if (blocks) {
        if (int_mode)
            hipLaunchKernelGGL(k_fill_seq_sparse<true>, dim3(blocks), dim3(kBlock), 0, st, a, w, idx,
                               pidx, syn_offsets, syn_targets, out, int_rescaler);
        else
            hipLaunchKernelGGL(k_fill_seq_sparse<false>, dim3(blocks), dim3(kBlock), 0, st, a, w, idx,
                               pidx, syn_offsets, syn_targets, out, int_rescaler);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (!int_mode) return hipSuccess;
    return launch_convert_i2f(out, (uint64_t)s.batch * s.seq * s.n_outputs, int_rescaler, st);
}

hipError_t launch_backward_seq_sparse(const SeqShape &s, uint32_t max_groups, const float *w,
                                      const float *g, const int32_t *anchors, const int32_t *idx,
                                      const float *md, const int32_t *mi, const int32_t *pidx,
                                      const float *pmd, const int32_t *pmi,
                                      const int64_t *syn_offsets, const int32_t *syn_targets,
                                      uint64_t n_synapses, float *x_grad, float *pe_grad,
                                      float *target, double lr, bool overwrite, bool int_mode,
                                      double int_rescaler, hipStream_t st) {
    const SeqSparseArgs a = make_args(s, max_groups);
    uint32_t blocks = 0;
    if (!grid_for(a, blocks)) return hipErrorInvalidConfiguration;
    const int2 *ap = reinterpret_cast<const int2 *>(anchors);
    hipError_t e = hipSuccess;
    // the weight gradient first: in the Internal policy the target is the
    // weights themselves, and the input gradient must see them unchanged --
    // so that case runs it last
    const bool internal = target == w;
    auto wgrad = [&]() -> hipError_t {
        if (!target) return hipSuccess;
        if (overwrite) {
            hipError_t z = launch_zero(target, n_synapses, st);
            if (z != hipSuccess) return z;
        }
        if (blocks) {
            if (int_mode)
                hipLaunchKernelGGL(k_wgrad_seq_sparse<true>, dim3(blocks), dim3(kBlock), 0, st, a, g, idx,
                                   pidx, syn_offsets, syn_targets, target, lr, int_rescaler);
            else
                hipLaunchKernelGGL(k_wgrad_seq_sparse<false>, dim3(blocks), dim3(kBlock), 0, st, a, g,
                                   idx, pidx, syn_offsets, syn_targets, target, lr, int_rescaler);
            hipError_t z = hipGetLastError();
            if (z != hipSuccess) return z;
        }
        if (int_mode) return launch_convert_i2f(target, n_synapses, int_rescaler, st);
        return hipSuccess;
    };
    if (!internal && (e = wgrad()) != hipSuccess) return e;
    if (blocks) {
        if (int_mode)
            hipLaunchKernelGGL(k_propagate_seq_sparse<true>, dim3(blocks), dim3(kBlock), 0, st, a, w, g,
                               idx, md, mi, pidx, pmd, pmi, ap, syn_offsets, syn_targets, x_grad,
                               pe_grad, int_rescaler);
        else
            hipLaunchKernelGGL(k_propagate_seq_sparse<false>, dim3(blocks), dim3(kBlock), 0, st, a, w, g,
                               idx, md, mi, pidx, pmd, pmi, ap, syn_offsets, syn_targets, x_grad,
                               pe_grad, int_rescaler);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (int_mode) {
        e = launch_convert_i2f(x_grad, (uint64_t)s.batch * s.seq * s.n_inputs, int_rescaler, st);
        if (e != hipSuccess) return e;
        if (s.pe_dim && pe_grad) {
            e = launch_convert_i2f(pe_grad, (uint64_t)(s.seq - 1) * s.n_detectors * s.pe_dim,
                                   int_rescaler, st);
            if (e != hipSuccess) return e;
        }
    }
    if (internal) return wgrad();
    return hipSuccess;
}

}  // namespace spiky
