/*
 * lut_oracle.c -- CPU restatement of the reference's LUT hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests and
 * bench.py's cpu_baseline leg use.  Nothing in the product (spiky_amd/) links,
 * loads or calls it.
 *
 * Every function restates the reference's NO_CUDA (device == -1) semantics:
 * the kernel body runs in serial loops blockIdx.y -> blockIdx.x -> threadIdx.x
 * (spiky_cuda/misc/misc.h:119-129), so a flat item index i = blockIdx.x*TPB +
 * threadIdx.x is visited in ascending order for every batch row in turn.  The
 * arithmetic (fp64 partial sums, fp32 commits, int32 fixed-point payloads) and
 * the rounding points follow the cited lines exactly.
 *
 * Pinning (what checks these functions independently of this file) is listed
 * per function in tests/test_oracle_*.py; functions with no such check say
 * "parity unpinned" here.
 *
 * Types: anchors are int32 pairs [n_detectors][n_anchors][2]; the value -1
 * (0xFFFFFFFF) marks an unused pair, as NeuronIndex_t max does in the
 * reference (lut_runtime_kernels_logic.proto:1076-1079).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* spiky_cuda/misc/misc.h:90 */
#define OR_EPS 0.00000000000000001
/* spiky_cuda/misc/misc.h:98-99 */
#define OR_DENOM32 1048575.0
#define OR_DENOM32_RECIPROC 9.536752259018191e-07

/* ROUNDED_COMPARISON_GREATER(delta, 0.0, cmp_eps), misc.h:16 */
static inline int rounded_greater0(float d, float cmp_eps)
{
    if (cmp_eps == 0.0f) return d > 0.0f;
    return (fabsf(d) < cmp_eps) ? 0 : (d > 0.0f);
}

/* int32 add with two's-complement wrap (what atomicAdd on int does, and what
 * the CPU build's `+=` produces on x86 in practice). */
static inline int32_t wrap_add(int32_t a, int32_t b)
{
    return (int32_t)((uint32_t)a + (uint32_t)b);
}

static inline int32_t *as_i32(float *p) { return (int32_t *)(void *)p; }

/* ------------------------------------------------------------------------ */
/* Anchor decode, compact mode: lut_compile_time_kernels_logic.proto:70-125. */
/* inputs_of_detector: CSR (offsets[n_det+1], ids[]) of each detector's      */
/* ascending input list (the CPU order of the backward synapse list).        */
/* Returns the number of detectors with <= 1 input (the reference's error    */
/* counter, lut.cu:537-550); such detectors are left untouched.              */
/* ------------------------------------------------------------------------ */
int64_t oracle_decode_anchors_compact(
    const uint32_t *encoded_pairs, int64_t n_detectors, int64_t max_pairs_per_detector,
    int64_t n_anchors, const int64_t *in_offsets, const int32_t *in_ids,
    int32_t *anchors_out)
{
    int64_t errors = 0;
    for (int64_t i = 0; i < n_detectors; i++) {
        const uint32_t *codes = encoded_pairs + i * max_pairs_per_detector;
        int32_t *dst = anchors_out + i * n_anchors * 2;
        uint32_t n_syn = (uint32_t)(in_offsets[i + 1] - in_offsets[i]);
        const int32_t *ids = in_ids + in_offsets[i];
        if (n_syn <= 1) { errors++; continue; }
        uint32_t max_codes = n_syn * (n_syn - 1);
        for (int64_t j = 0; j < n_anchors; j++) {
            uint32_t c = codes[j] % max_codes;
            uint32_t a1 = c / (n_syn - 1);
            uint32_t a2 = c % (n_syn - 1);
            if (a2 >= a1) a2++;
            dst[2 * j] = ids[a1];
            dst[2 * j + 1] = ids[a2];
        }
    }
    return errors;
}

/* ------------------------------------------------------------------------ */
/* check_detectors_logic (train) proto:1099-1158 and check_detectors_eval    */
/* proto:1050-1097.  w_min_deltas == NULL selects eval.                      */
/* ------------------------------------------------------------------------ */
void oracle_check_detectors(
    const float *x, int64_t batch, int64_t n_inputs,
    const int32_t *anchors, int64_t n_detectors, int64_t n_anchors, float cmp_eps,
    int32_t *w_idx, float *w_min_deltas, int32_t *w_min_idx)
{
    for (int64_t b = 0; b < batch; b++) {
        const float *xb = x + b * n_inputs;
        for (int64_t t = 0; t < n_detectors; t++) {
            const int32_t *ap = anchors + t * n_anchors * 2;
            int32_t li = 0;
            float md = 0.0f;
            int32_t mi = -1;
            for (int64_t k = 0; k < n_anchors; k++) {
                int32_t a1 = ap[2 * k], a2 = ap[2 * k + 1];
                if (a1 == -1 || a2 == -1) continue;
                float d = xb[a1] - xb[a2];
                if (rounded_greater0(d, cmp_eps)) li |= (1 << k);
                if (mi == -1 || fabsf(d) < fabsf(md)) { md = d; mi = (int32_t)k; }
            }
            w_idx[b * n_detectors + t] = li;
            if (w_min_deltas) {
                w_min_deltas[b * n_detectors + t] = md;
                w_min_idx[b * n_detectors + t] = mi;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* fill_outputs_non_seq_fc_logic, proto:1214-1299.  Item i = blk*O + o, so   */
/* for each sample the blocks of `dgs` detectors are committed in ascending  */
/* block order.  Each block: fp64 sum of the selected weights in ascending   */
/* detector order, then one fp32 commit (float mode) or one int32 payload    */
/* trunc(sum*DENOM32*int_rescaler) (int mode, proto:1276-1285).              */
/* W layout [n_detectors][n_entries][O] (row = t*E + idx), proto:1233-1270.  */
/* If q8 != NULL the table is int8 with a per-detector fp32 scale and the    */
/* weight is the fp32 product scale[t]*(float)q (the int8 mapping of the     */
/* integer path; the reference itself stores fp32 weights only).             */
/* ------------------------------------------------------------------------ */
static inline double weight_at(const float *w, const int8_t *q8, const float *scales,
                               int64_t t, int64_t off)
{
    if (q8) return (double)(scales[t] * (float)q8[off]);
    return (double)w[off];
}

void oracle_fill_outputs_fc(
    const float *w, const int8_t *q8, const float *scales,
    const int32_t *idx, float *out, int64_t batch, int64_t n_outputs,
    int64_t n_detectors, int64_t n_entries, int64_t dgs, int int_mode, double int_rescaler)
{
    int64_t n_blocks = (n_detectors + dgs - 1) / dgs;
    for (int64_t b = 0; b < batch; b++) {
        const int32_t *ib = idx + b * n_detectors;
        float *ob = out + b * n_outputs;
        for (int64_t blk = 0; blk < n_blocks; blk++) {
            int64_t t0 = blk * dgs;
            int64_t t1 = t0 + dgs < n_detectors ? t0 + dgs : n_detectors;
            for (int64_t o = 0; o < n_outputs; o++) {
                double s = 0.0;
                for (int64_t t = t0; t < t1; t++) {
                    int64_t off = (t * n_entries + ib[t]) * n_outputs + o;
                    s += weight_at(w, q8, scales, t, off);
                }
                if (int_mode) {
                    int32_t p = (int32_t)(s * OR_DENOM32 * int_rescaler);
                    as_i32(ob)[o] = wrap_add(as_i32(ob)[o], p);
                } else {
                    ob[o] += (float)s;
                }
            }
        }
    }
}

/* convert_integers_to_floats_logic, proto:200-213: in-place int32 -> fp32. */
void oracle_convert_int_to_float(float *buf, int64_t n, double int_rescaler)
{
    for (int64_t i = 0; i < n; i++) {
        double y = (double)as_i32(buf)[i] * OR_DENOM32_RECIPROC;
        buf[i] = (float)(y / int_rescaler);
    }
}

/* du = sign(u)*0.5/(1+|u|)^2 with sign(u<=0) = -1, evaluated as the         */
/* reference does: proto:1458-1465.                                          */
static inline double du_of_margin(float md)
{
    double du = (double)md;
    if (du > 0) {
        du = 1.0 / (1.0 + fabs(du));
        du *= 0.5 * du;
    } else {
        du = 1.0 / (1.0 + fabs(du));
        du *= -0.5 * du;
    }
    return du;
}

/* propagate_through_detector, proto:821-867 (CPU branch). */
static inline void push_input_grad(float *xg, int32_t a1, int32_t a2, double du,
                                   int int_mode, double int_rescaler)
{
    if (!(fabs(du) > OR_EPS)) return;
    if (int_mode) {
        int32_t d = (int32_t)(du * OR_DENOM32 * int_rescaler);
        as_i32(xg)[a1] = wrap_add(as_i32(xg)[a1], d);
        as_i32(xg)[a2] = wrap_add(as_i32(xg)[a2], (int32_t)(0u - (uint32_t)d));
    } else {
        /* float += double: one rounding through double (C semantics) */
        xg[a1] = (float)((double)xg[a1] + du);
        xg[a2] = (float)((double)xg[a2] - du);
    }
}

/* ------------------------------------------------------------------------ */
/* propagate_through_detectors_non_seq_fc_logic, proto:1421-1499, with       */
/* accumulate_pair_of_gradient_sums_fc proto:474-582 (CPU branch 575-581).   */
/* Item i = t*n_ob + ob.  A detector whose min-index is -1 (no valid anchor) */
/* contributes nothing (the reference shifts by -1 there, which is UB).      */
/* ------------------------------------------------------------------------ */
void oracle_propagate_fc(
    const float *w, const float *g, const int32_t *idx, const float *min_deltas,
    const int32_t *min_idx, const int32_t *anchors, float *x_grad,
    int64_t batch, int64_t n_inputs, int64_t n_outputs, int64_t n_detectors,
    int64_t n_anchors, int64_t n_entries, int64_t ogs, int int_mode, double int_rescaler)
{
    int64_t n_ob = (n_outputs + ogs - 1) / ogs;
    for (int64_t b = 0; b < batch; b++) {
        const float *gb = g + b * n_outputs;
        float *xg = x_grad + b * n_inputs;
        for (int64_t t = 0; t < n_detectors; t++) {
            int32_t li = idx[b * n_detectors + t];
            int32_t mi = min_idx[b * n_detectors + t];
            float md = min_deltas[b * n_detectors + t];
            for (int64_t ob = 0; ob < n_ob; ob++) {
                if (mi < 0) continue;
                double du = du_of_margin(md);
                int64_t main_row = t * n_entries + li;
                int64_t alt_row = t * n_entries + (li ^ (1 << mi));
                int64_t o0 = ob * ogs;
                int64_t o1 = o0 + ogs < n_outputs ? o0 + ogs : n_outputs;
                double ms = 0.0, as = 0.0;
                for (int64_t o = o0; o < o1; o++) {
                    double gg = (double)gb[o];
                    ms += (double)w[main_row * n_outputs + o] * gg;
                    as += (double)w[alt_row * n_outputs + o] * gg;
                }
                du *= ms - as;
                const int32_t *ap = anchors + (t * n_anchors + mi) * 2;
                push_input_grad(xg, ap[0], ap[1], du, int_mode, int_rescaler);
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* gather_w_gradients_non_seq_fc_logic proto:1547-1585 with                  */
/* gather_weight_gradients_fc proto:716-819 (CPU branch 792-818).            */
/* lr = (double)first_meta_lr, times -external_lr when external_lr >= 0      */
/* (then `target` is the weight tensor itself: in-place SGD,                 */
/* lut_runtime.cu:342-361).                                                  */
/* ------------------------------------------------------------------------ */
void oracle_gather_wgrad_fc(
    const float *g, const int32_t *idx, float *target,
    int64_t batch, int64_t n_outputs, int64_t n_detectors, int64_t n_entries, int64_t ogs,
    float first_meta_lr, float external_lr, int int_mode, double int_rescaler)
{
    int64_t n_ob = (n_outputs + ogs - 1) / ogs;
    double lr = (double)first_meta_lr;
    if (external_lr >= 0) lr *= -(double)external_lr;
    for (int64_t b = 0; b < batch; b++) {
        const float *gb = g + b * n_outputs;
        for (int64_t t = 0; t < n_detectors; t++) {
            int64_t row = t * n_entries + idx[b * n_detectors + t];
            for (int64_t ob = 0; ob < n_ob; ob++) {
                int64_t o0 = ob * ogs;
                int64_t o1 = o0 + ogs < n_outputs ? o0 + ogs : n_outputs;
                for (int64_t o = o0; o < o1; o++) {
                    double gg = (double)gb[o];
                    if (!(fabs(gg) > OR_EPS)) continue;
                    if (int_mode) {
                        int32_t d = (int32_t)(gg * lr * OR_DENOM32 * int_rescaler);
                        as_i32(target)[row * n_outputs + o] =
                            wrap_add(as_i32(target)[row * n_outputs + o], d);
                    } else {
                        target[row * n_outputs + o] += (float)(gg * lr);
                    }
                }
            }
        }
    }
}

/* ======================================================================== */
/* Sparse (ProjectionLUTLayer) path over this build's CSR layout:            */
/*   syn_offsets[n_lookup+1]  - synapses of lookup neuron n = t*E + e        */
/*   syn_targets[n_syn]       - output index of each synapse                 */
/*   weights[n_syn]           - one fp32 weight per synapse                  */
/* A neuron's synapses split into forward groups of `fgs` in list order      */
/* (the reference's ForwardSynapseGroup, connections_manager.h:39-66).       */
/* ======================================================================== */

/* fill_outputs_non_seq_sparse_logic proto:1160-1212 + fire_single_synapse_group
 * proto:215-313: per synapse one fp32 commit of (float)(double)w, items ordered
 * (t, group) ascending, synapses in list order. */
void oracle_fill_outputs_sparse(
    const float *w, const int32_t *idx, const int64_t *syn_offsets, const int32_t *syn_targets,
    float *out, int64_t batch, int64_t n_outputs, int64_t n_detectors, int64_t n_entries,
    int int_mode, double int_rescaler)
{
    for (int64_t b = 0; b < batch; b++) {
        float *ob = out + b * n_outputs;
        for (int64_t t = 0; t < n_detectors; t++) {
            int64_t n = t * n_entries + idx[b * n_detectors + t];
            for (int64_t s = syn_offsets[n]; s < syn_offsets[n + 1]; s++) {
                int32_t tg = syn_targets[s];
                double wt = (double)w[s];
                if (int_mode) {
                    int32_t p = (int32_t)(wt * OR_DENOM32 * int_rescaler);
                    as_i32(ob)[tg] = wrap_add(as_i32(ob)[tg], p);
                } else {
                    ob[tg] += (float)wt;
                }
            }
        }
    }
}

/* propagate_through_detectors_non_seq_sparse_logic proto:1303-1419 with
 * accumulate_grad_sum_sparse proto:315-395.  Group `grp` of the main neuron
 * and group `grp` of the alt neuron (each only if it exists), then one du per
 * (t, grp), grp < max_groups. */
void oracle_propagate_sparse(
    const float *w, const float *g, const int32_t *idx, const float *min_deltas,
    const int32_t *min_idx, const int32_t *anchors, const int64_t *syn_offsets,
    const int32_t *syn_targets, float *x_grad, int64_t batch, int64_t n_inputs,
    int64_t n_outputs, int64_t n_detectors, int64_t n_anchors, int64_t n_entries,
    int64_t fgs, int64_t max_groups, int int_mode, double int_rescaler)
{
    for (int64_t b = 0; b < batch; b++) {
        const float *gb = g + b * n_outputs;
        float *xg = x_grad + b * n_inputs;
        for (int64_t t = 0; t < n_detectors; t++) {
            int32_t li = idx[b * n_detectors + t];
            int32_t mi = min_idx[b * n_detectors + t];
            float md = min_deltas[b * n_detectors + t];
            for (int64_t grp = 0; grp < max_groups; grp++) {
                if (mi < 0) continue;
                double du = du_of_margin(md);
                int64_t nm = t * n_entries + li;
                int64_t na = t * n_entries + (li ^ (1 << mi));
                double ms = 0.0, as = 0.0;
                int64_t s0 = syn_offsets[nm] + grp * fgs;
                if (s0 < syn_offsets[nm + 1]) {
                    int64_t s1 = s0 + fgs < syn_offsets[nm + 1] ? s0 + fgs : syn_offsets[nm + 1];
                    for (int64_t s = s0; s < s1; s++)
                        ms += (double)w[s] * (double)gb[syn_targets[s]];
                }
                s0 = syn_offsets[na] + grp * fgs;
                if (s0 < syn_offsets[na + 1]) {
                    int64_t s1 = s0 + fgs < syn_offsets[na + 1] ? s0 + fgs : syn_offsets[na + 1];
                    for (int64_t s = s0; s < s1; s++)
                        as += (double)w[s] * (double)gb[syn_targets[s]];
                }
                du *= ms - as;
                const int32_t *ap = anchors + (t * n_anchors + mi) * 2;
                push_input_grad(xg, ap[0], ap[1], du, int_mode, int_rescaler);
            }
        }
    }
}

/* gather_w_gradients_non_seq_sparse_logic proto:1501-1545 with
 * gather_weight_gradients_sparse proto:584-714. */
void oracle_gather_wgrad_sparse(
    const float *g, const int32_t *idx, const int64_t *syn_offsets, const int32_t *syn_targets,
    float *target, int64_t batch, int64_t n_outputs, int64_t n_detectors, int64_t n_entries,
    float first_meta_lr, float external_lr, int int_mode, double int_rescaler)
{
    double lr = (double)first_meta_lr;
    if (external_lr >= 0) lr *= -(double)external_lr;
    for (int64_t b = 0; b < batch; b++) {
        const float *gb = g + b * n_outputs;
        for (int64_t t = 0; t < n_detectors; t++) {
            int64_t n = t * n_entries + idx[b * n_detectors + t];
            for (int64_t s = syn_offsets[n]; s < syn_offsets[n + 1]; s++) {
                double gg = (double)gb[syn_targets[s]];
                if (!(fabs(gg) > OR_EPS)) continue;
                if (int_mode) {
                    int32_t d = (int32_t)(gg * lr * OR_DENOM32 * int_rescaler);
                    as_i32(target)[s] = wrap_add(as_i32(target)[s], d);
                } else {
                    target[s] += (float)(gg * lr);
                }
            }
        }
    }
}

/* ======================================================================== */
/* Sequence-concat mode (LUTTransformer attention).                          */
/* Layouts: x [B][S][I]; idx / md / mi [B][S][T]; pe [(S-1)][T][Npe];        */
/* pidx / pmd / pmi [(S-1)][T]; out / g [B][S][O];                           */
/* W [T][2^(2Nc+Npe)][O] with row (Q << (Nc+Npe)) | (K << Npe) | PE.         */
/* check_detectors_seq(_eval) (proto:1589-1707) is check_detectors over the  */
/* B*S rows of x, which is what the callers use.                             */
/* ======================================================================== */

/* check_positional_embeddings(_eval)_logic, proto:1709-1805.  pmd / pmi     */
/* may be NULL (eval).                                                       */
void oracle_check_pe(
    const float *pe, int64_t seq_len, int64_t n_detectors, int64_t positional_dim,
    float cmp_eps, int32_t *pidx, float *pmd, int32_t *pmi)
{
    for (int64_t it = 0; it < (seq_len - 1) * n_detectors; it++) {
        const float *v = pe + it * positional_dim;
        int32_t li = 0, mk = -1;
        float mind = 0.0f;
        for (int64_t d = 0; d < positional_dim; d++) {
            if (rounded_greater0(v[d], cmp_eps)) li |= (1 << d);
            if (mk == -1 || fabsf(v[d]) < fabsf(mind)) {
                mind = v[d];
                mk = (int32_t)d;
            }
        }
        pidx[it] = li;
        if (pmd) pmd[it] = mind;
        if (pmi) pmi[it] = mk;
    }
}

static inline int64_t seq_row(int32_t q, int32_t k, int32_t p, int64_t n_anchors, int64_t pd)
{
    return ((int64_t)q << (n_anchors + pd)) | ((int64_t)k << pd) | (int64_t)p;
}

/* fill_outputs_fully_connected_seq_logic, proto:1807-1904.  Serial order:   */
/* for b: item ((j-1)*T + t)*O + o ascending; each item commits the fp64 sum */
/* over i < j once (fp32, or the int32 payload).                             */
void oracle_fill_outputs_seq(
    const float *w, const int32_t *idx, const int32_t *pidx, float *out,
    int64_t batch, int64_t n_outputs, int64_t n_detectors, int64_t seq_len,
    int64_t n_anchors, int64_t positional_dim, int int_mode, double int_rescaler)
{
    const int64_t nlpd = (int64_t)1 << (2 * n_anchors + positional_dim);
    for (int64_t b = 0; b < batch; b++) {
        for (int64_t j = 1; j < seq_len; j++) {
            for (int64_t t = 0; t < n_detectors; t++) {
                int32_t q = idx[(b * seq_len + j) * n_detectors + t];
                for (int64_t o = 0; o < n_outputs; o++) {
                    double ws = 0.0;
                    for (int64_t i = 0; i < j; i++) {
                        int32_t k = idx[(b * seq_len + i) * n_detectors + t];
                        int32_t p = positional_dim > 0 ? pidx[(j - i - 1) * n_detectors + t] : 0;
                        int64_t row = t * nlpd + seq_row(q, k, p, n_anchors, positional_dim);
                        ws += (double)w[row * n_outputs + o];
                    }
                    float *dst = out + (b * seq_len + j) * n_outputs + o;
                    if (int_mode)
                        *as_i32(dst) = wrap_add(*as_i32(dst), (int32_t)(ws * OR_DENOM32 * int_rescaler));
                    else
                        *dst += (float)ws;
                }
            }
        }
    }
}

/* Visits the causal pairs in the reference CPU path's serial order for the  */
/* seq backward kernels (lut_runtime.cu:630-637, proto:3653-3689):           */
/* b -> output block -> tile (ti row-major, tiles with ti > tj skipped) ->   */
/* detector -> thread (i = ti*32 + tid%32, j = tj*32 + tid/32, i < j).       */
#define OR_TILE 32
#define FOR_SEQ_PAIRS(B, S, NOB, T, ...)                                               \
    do {                                                                               \
        int64_t tgw_ = ((S) + OR_TILE - 1) / OR_TILE;                                  \
        for (int64_t b = 0; b < (B); b++)                                              \
            for (int64_t ob = 0; ob < (NOB); ob++)                                     \
                for (int64_t tile_ = 0; tile_ < tgw_ * tgw_; tile_++) {                \
                    int64_t ti_ = tile_ / tgw_, tj_ = tile_ % tgw_;                    \
                    if (ti_ > tj_) continue;                                           \
                    for (int64_t t = 0; t < (T); t++)                                  \
                        for (int64_t tid_ = 0; tid_ < OR_TILE * OR_TILE; tid_++) {     \
                            int64_t i = ti_ * OR_TILE + tid_ % OR_TILE;                \
                            int64_t j = tj_ * OR_TILE + tid_ / OR_TILE;                \
                            if (i >= j || j >= (S)) continue;                          \
                            __VA_ARGS__                                                \
                        }                                                              \
                }                                                                      \
    } while (0)

static inline double block_dot(const float *w, int64_t row, const float *gj, int64_t n_outputs,
                               int64_t o0, int64_t o1)
{
    double s = 0.0;
    for (int64_t o = o0; o < o1; o++) s += (double)w[row * n_outputs + o] * (double)gj[o];
    return s;
}

/* propagate_through_detectors_seq_fc_logic, proto:3629-3835, with           */
/* accumulate_pair_of_gradient_sums_fc / accumulate_grad_sum_fc (proto:396-  */
/* 582), propagate_through_detector (proto:821-867) and                      */
/* update_positional_gradients (proto:1016-1046, no EPS cut).  Per (pair,    */
/* detector, output block): flip Q's min anchor if |dQ| < |dK| else K's; the */
/* positional flip applies when |dPE| is strictly the smallest.  pe_grad may */
/* be NULL when positional_dim == 0.                                         */
/* x_grad64 / pe_grad64 (fp32 summation only, may be null): when given, the */
/* same terms (same EPS cut) are accumulated there in fp64 instead of into   */
/* the fp32 buffers -- the reference's sums without its fp32 rounding of     */
/* every partial sum, to check a device path that rounds fewer times.        */
void oracle_propagate_seq(
    const float *w, const float *g, const int32_t *idx, const float *md, const int32_t *mi,
    const int32_t *pidx, const float *pmd, const int32_t *pmi, const int32_t *anchors,
    float *x_grad, float *pe_grad, int64_t batch, int64_t n_inputs, int64_t n_outputs,
    int64_t n_detectors, int64_t seq_len, int64_t n_anchors, int64_t positional_dim, int64_t ogs,
    int int_mode, double int_rescaler, double *x_grad64, double *pe_grad64)
{
    const int64_t nlpd = (int64_t)1 << (2 * n_anchors + positional_dim);
    const int64_t n_ob = (n_outputs + ogs - 1) / ogs;
    const int64_t pd = positional_dim;
    FOR_SEQ_PAIRS(batch, seq_len, n_ob, n_detectors, {
        int64_t o0 = ob * ogs, o1 = o0 + ogs < n_outputs ? o0 + ogs : n_outputs;
        int64_t ko = (b * seq_len + i) * n_detectors + t, qo = (b * seq_len + j) * n_detectors + t;
        int32_t K = idx[ko], Q = idx[qo];
        int32_t km = mi[ko], qm = mi[qo];
        float kd = md[ko], qd = md[qo];
        int32_t P = 0, pm = -1;
        float pdl = 0.0f;
        int64_t pe_off = (j - i - 1) * n_detectors + t;
        if (pd > 0) {
            P = pidx[pe_off];
            pm = pmi[pe_off];
            pdl = pmd[pe_off];
        }
        const float *gj = g + (b * seq_len + j) * n_outputs;
        int64_t main_row = t * nlpd + seq_row(Q, K, P, n_anchors, pd);
        int64_t alt_row, src_pos;
        int32_t flip;
        double du;
        if (fabsf(qd) < fabsf(kd)) {
            alt_row = t * nlpd + seq_row(qm >= 0 ? Q ^ (1 << qm) : Q, K, P, n_anchors, pd);
            du = du_of_margin(qd);
            flip = qm;
            src_pos = j;
        } else {
            alt_row = t * nlpd + seq_row(Q, km >= 0 ? K ^ (1 << km) : K, P, n_anchors, pd);
            du = du_of_margin(kd);
            flip = km;
            src_pos = i;
        }
        double ms = block_dot(w, main_row, gj, n_outputs, o0, o1);
        double as = block_dot(w, alt_row, gj, n_outputs, o0, o1);
        du *= ms - as;
        if (flip >= 0) {
            const int32_t *ap = anchors + (t * n_anchors + flip) * 2;
            if (x_grad64 && !int_mode) {
                double *xg = x_grad64 + (b * seq_len + src_pos) * n_inputs;
                if (fabs(du) > OR_EPS) {
                    xg[ap[0]] += du;
                    xg[ap[1]] -= du;
                }
            } else {
                push_input_grad(x_grad + (b * seq_len + src_pos) * n_inputs, ap[0], ap[1], du, int_mode,
                                int_rescaler);
            }
        }
        if (pd > 0 && fabsf(pdl) < fabsf(qd) && fabsf(pdl) < fabsf(kd) && pm >= 0) {
            int64_t pe_row = t * nlpd + seq_row(Q, K, P ^ (1 << pm), n_anchors, pd);
            double dpe = du_of_margin(pdl) * (ms - block_dot(w, pe_row, gj, n_outputs, o0, o1));
            float *dst = pe_grad + pe_off * pd + pm;
            if (pe_grad64 && !int_mode)
                pe_grad64[pe_off * pd + pm] += dpe;
            else if (int_mode)
                *as_i32(dst) = wrap_add(*as_i32(dst), (int32_t)(dpe * OR_DENOM32 * int_rescaler));
            else
                *dst = (float)((double)*dst + dpe);
        }
    });
}

/* gather_w_gradients_seq_fc_cpu_logic, proto:3944-4045, with                */
/* gather_weight_gradients_fc (proto:716-819, CPU branch 792-818): every     */
/* causal pair (i < j) adds (float)(g[b][j][o] * lr) to its row (|g| > EPS). */
void oracle_gather_wgrad_seq(
    const float *g, const int32_t *idx, const int32_t *pidx, float *target,
    int64_t batch, int64_t n_outputs, int64_t n_detectors, int64_t seq_len, int64_t n_anchors,
    int64_t positional_dim, int64_t ogs, float first_meta_lr, float external_lr, int int_mode,
    double int_rescaler)
{
    const int64_t nlpd = (int64_t)1 << (2 * n_anchors + positional_dim);
    const int64_t n_ob = (n_outputs + ogs - 1) / ogs;
    double lr = (double)first_meta_lr;
    if (external_lr >= 0) lr *= -(double)external_lr;
    FOR_SEQ_PAIRS(batch, seq_len, n_ob, n_detectors, {
        int64_t o0 = ob * ogs, o1 = o0 + ogs < n_outputs ? o0 + ogs : n_outputs;
        int32_t K = idx[(b * seq_len + i) * n_detectors + t];
        int32_t Q = idx[(b * seq_len + j) * n_detectors + t];
        int32_t P = positional_dim > 0 ? pidx[(j - i - 1) * n_detectors + t] : 0;
        int64_t row = t * nlpd + seq_row(Q, K, P, n_anchors, positional_dim);
        const float *gj = g + (b * seq_len + j) * n_outputs;
        for (int64_t o = o0; o < o1; o++) {
            double gg = (double)gj[o];
            if (!(fabs(gg) > OR_EPS)) continue;
            float *dst = target + row * n_outputs + o;
            if (int_mode)
                *as_i32(dst) = wrap_add(*as_i32(dst), (int32_t)(gg * lr * OR_DENOM32 * int_rescaler));
            else
                *dst += (float)(gg * lr);
        }
    });
}

/* ------------------------------------------------------------------------ */
/* Sequence-concat over sparse lookup connectivity (this build's CSR: lookup */
/* neuron n owns synapses [syn_offsets[n], syn_offsets[n+1]), forward group  */
/* g = its synapses g*fgs .. g*fgs+fgs-1 in list order; W is per synapse).   */
/* fill_outputs_sparse_seq_logic (proto:1906-2015),                          */
/* propagate_through_detectors_seq_sparse_logic (proto:3371-3627) and        */
/* gather_w_gradients_seq_sparse_logic (proto:3837-3942) in the serial order */
/* of the reference CPU path: (b, group) -> (32x32 tile, detector) -> tile   */
/* thread, whose pair is i = ti*32 + tid/32, j = tj*32 + tid%32 (these       */
/* kernels index the tile the other way round from the FC ones).             */
/* ------------------------------------------------------------------------ */
#define FOR_SEQ_PAIRS_SPARSE(B, S, NOB, T, ...)                                        \
    do {                                                                               \
        int64_t tgw_ = ((S) + OR_TILE - 1) / OR_TILE;                                  \
        for (int64_t b = 0; b < (B); b++)                                              \
            for (int64_t ob = 0; ob < (NOB); ob++)                                     \
                for (int64_t tile_ = 0; tile_ < tgw_ * tgw_; tile_++) {                \
                    int64_t ti_ = tile_ / tgw_, tj_ = tile_ % tgw_;                    \
                    if (ti_ > tj_) continue;                                           \
                    for (int64_t t = 0; t < (T); t++)                                  \
                        for (int64_t tid_ = 0; tid_ < OR_TILE * OR_TILE; tid_++) {     \
                            int64_t i = ti_ * OR_TILE + tid_ / OR_TILE;                \
                            int64_t j = tj_ * OR_TILE + tid_ % OR_TILE;                \
                            if (i >= j || j >= (S)) continue;                          \
                            __VA_ARGS__                                                \
                        }                                                              \
                }                                                                      \
    } while (0)

/* synapses of forward group ob of neuron n: [*s0, *s1), empty if absent */
static inline void group_range(const int64_t *syn_offsets, int64_t n, int64_t ob, int64_t fgs,
                               int64_t *s0, int64_t *s1)
{
    *s0 = syn_offsets[n] + ob * fgs;
    *s1 = *s0 + fgs < syn_offsets[n + 1] ? *s0 + fgs : syn_offsets[n + 1];
    if (*s0 > *s1) *s0 = *s1;
}

static inline double group_dot(const float *w, const int64_t *syn_offsets, const int32_t *syn_targets,
                               int64_t n, int64_t ob, int64_t fgs, const float *gj)
{
    int64_t s0, s1;
    double acc = 0.0;
    group_range(syn_offsets, n, ob, fgs, &s0, &s1);
    for (int64_t s = s0; s < s1; s++) acc += (double)w[s] * (double)gj[syn_targets[s]];
    return acc;
}

/* out [B][S][O]: each synapse of the pair's group commits (float)(double)w  */
/* (fire_single_synapse_group, proto:215-313), or its int32 payload.          */
void oracle_fill_outputs_seq_sparse(
    const float *w, const int32_t *idx, const int32_t *pidx, const int64_t *syn_offsets,
    const int32_t *syn_targets, float *out, int64_t batch, int64_t seq_len, int64_t n_outputs,
    int64_t n_detectors, int64_t n_anchors, int64_t positional_dim, int64_t fgs, int64_t max_groups,
    int int_mode, double int_rescaler)
{
    const int64_t nlpd = (int64_t)1 << (2 * n_anchors + positional_dim);
    FOR_SEQ_PAIRS_SPARSE(batch, seq_len, max_groups, n_detectors, {
        int32_t K = idx[(b * seq_len + i) * n_detectors + t];
        int32_t Q = idx[(b * seq_len + j) * n_detectors + t];
        int32_t P = positional_dim > 0 ? pidx[(j - i - 1) * n_detectors + t] : 0;
        int64_t n = t * nlpd + seq_row(Q, K, P, n_anchors, positional_dim);
        int64_t s0, s1;
        group_range(syn_offsets, n, ob, fgs, &s0, &s1);
        float *oj = out + (b * seq_len + j) * n_outputs;
        for (int64_t s = s0; s < s1; s++) {
            int32_t tg = syn_targets[s];
            double wt = (double)w[s];
            if (int_mode)
                as_i32(oj)[tg] = wrap_add(as_i32(oj)[tg], (int32_t)(wt * OR_DENOM32 * int_rescaler));
            else
                oj[tg] += (float)wt;
        }
    });
}

/* As oracle_propagate_seq over the pair's group ob of the main, flipped and */
/* PE-flipped neurons.  x_sum / x_abs / pe_sum / pe_abs (fp32 summation,     */
/* may be null): when given, the pushes are also accumulated there in fp64   */
/* with their magnitudes -- the bound for a device path that adds the same   */
/* terms in another order.                                                   */
void oracle_propagate_seq_sparse(
    const float *w, const float *g, const int32_t *idx, const float *md, const int32_t *mi,
    const int32_t *pidx, const float *pmd, const int32_t *pmi, const int32_t *anchors,
    const int64_t *syn_offsets, const int32_t *syn_targets, float *x_grad, float *pe_grad,
    int64_t batch, int64_t n_inputs, int64_t n_outputs, int64_t n_detectors, int64_t seq_len,
    int64_t n_anchors, int64_t positional_dim, int64_t fgs, int64_t max_groups, int int_mode,
    double int_rescaler, double *x_sum, double *x_abs, double *pe_sum, double *pe_abs)
{
    const int64_t nlpd = (int64_t)1 << (2 * n_anchors + positional_dim);
    const int64_t pd = positional_dim;
    FOR_SEQ_PAIRS_SPARSE(batch, seq_len, max_groups, n_detectors, {
        int64_t ko = (b * seq_len + i) * n_detectors + t, qo = (b * seq_len + j) * n_detectors + t;
        int32_t K = idx[ko], Q = idx[qo];
        int32_t km = mi[ko], qm = mi[qo];
        float kd = md[ko], qd = md[qo];
        int32_t P = 0, pm = -1;
        float pdl = 0.0f;
        int64_t pe_off = (j - i - 1) * n_detectors + t;
        if (pd > 0) {
            P = pidx[pe_off];
            pm = pmi[pe_off];
            pdl = pmd[pe_off];
        }
        const float *gj = g + (b * seq_len + j) * n_outputs;
        int64_t main_n = t * nlpd + seq_row(Q, K, P, n_anchors, pd);
        int64_t alt_n, src_pos;
        int32_t flip;
        double du;
        if (fabsf(qd) < fabsf(kd)) {
            alt_n = t * nlpd + seq_row(qm >= 0 ? Q ^ (1 << qm) : Q, K, P, n_anchors, pd);
            du = du_of_margin(qd);
            flip = qm;
            src_pos = j;
        } else {
            alt_n = t * nlpd + seq_row(Q, km >= 0 ? K ^ (1 << km) : K, P, n_anchors, pd);
            du = du_of_margin(kd);
            flip = km;
            src_pos = i;
        }
        double ms = group_dot(w, syn_offsets, syn_targets, main_n, ob, fgs, gj);
        double as = group_dot(w, syn_offsets, syn_targets, alt_n, ob, fgs, gj);
        du *= ms - as;
        if (flip >= 0) {
            const int32_t *ap = anchors + (t * n_anchors + flip) * 2;
            int64_t row = (b * seq_len + src_pos) * n_inputs;
            push_input_grad(x_grad + row, ap[0], ap[1], du, int_mode, int_rescaler);
            if (x_sum && fabs(du) > OR_EPS) {
                double f = (double)(float)du;
                x_sum[row + ap[0]] += f;
                x_abs[row + ap[0]] += fabs(f);
                x_sum[row + ap[1]] -= f;
                x_abs[row + ap[1]] += fabs(f);
            }
        }
        if (pd > 0 && fabsf(pdl) < fabsf(qd) && fabsf(pdl) < fabsf(kd) && pm >= 0) {
            int64_t pe_n = t * nlpd + seq_row(Q, K, P ^ (1 << pm), n_anchors, pd);
            double dpe = du_of_margin(pdl) * (ms - group_dot(w, syn_offsets, syn_targets, pe_n, ob, fgs, gj));
            float *dst = pe_grad + pe_off * pd + pm;
            if (int_mode)
                *as_i32(dst) = wrap_add(*as_i32(dst), (int32_t)(dpe * OR_DENOM32 * int_rescaler));
            else
                *dst = (float)((double)*dst + dpe);
            if (pe_sum) {
                double f = (double)(float)dpe;
                pe_sum[pe_off * pd + pm] += f;
                pe_abs[pe_off * pd + pm] += fabs(f);
            }
        }
    });
}

/* target [n_synapses]: every synapse of the pair's group adds                */
/* (float)(g[b][j][target] * lr) where |g| > EPS (gather_weight_gradients_sparse, */
/* proto:584-714).                                                            */
void oracle_gather_wgrad_seq_sparse(
    const float *g, const int32_t *idx, const int32_t *pidx, const int64_t *syn_offsets,
    const int32_t *syn_targets, float *target, int64_t batch, int64_t seq_len, int64_t n_outputs,
    int64_t n_detectors, int64_t n_anchors, int64_t positional_dim, int64_t fgs, int64_t max_groups,
    float first_meta_lr, float external_lr, int int_mode, double int_rescaler)
{
    const int64_t nlpd = (int64_t)1 << (2 * n_anchors + positional_dim);
    double lr = (double)first_meta_lr;
    if (external_lr >= 0) lr *= -(double)external_lr;
    FOR_SEQ_PAIRS_SPARSE(batch, seq_len, max_groups, n_detectors, {
        int32_t K = idx[(b * seq_len + i) * n_detectors + t];
        int32_t Q = idx[(b * seq_len + j) * n_detectors + t];
        int32_t P = positional_dim > 0 ? pidx[(j - i - 1) * n_detectors + t] : 0;
        int64_t n = t * nlpd + seq_row(Q, K, P, n_anchors, positional_dim);
        int64_t s0, s1;
        group_range(syn_offsets, n, ob, fgs, &s0, &s1);
        const float *gj = g + (b * seq_len + j) * n_outputs;
        for (int64_t s = s0; s < s1; s++) {
            double gg = (double)gj[syn_targets[s]];
            if (!(fabs(gg) > OR_EPS)) continue;
            if (int_mode)
                as_i32(target)[s] = wrap_add(as_i32(target)[s], (int32_t)(gg * lr * OR_DENOM32 * int_rescaler));
            else
                target[s] += (float)(gg * lr);
        }
    });
}

/* ------------------------------------------------------------------------ */
/* Product mode (concatenation_product == False): every causal pair i < j   */
/* of a sequence is one LUT lookup over the virtual input row               */
/* [x1[i] (n1) | x2[j] (n2) | pe[j-i-1][t] (pd)] (or, in sliced mode, the   */
/* interleaving x1[0] x2[0] pe[0] x1[1] ...), with per-detector positional  */
/* slices pe[(j-i-1)*T + t][pd].  Restated from                             */
/* calculate_product_lookup_index(_backprop), proto:32-181,                 */
/* fill_outputs_product_cpu_logic proto:2148-2264,                          */
/* propagate_backward_product_cpu_logic proto:2396-2628 with                */
/* propagate_through_detector_product proto:869-1023, accumulate_grad_sum_fc */
/* (CPU branch) proto:397-472 and gather_weight_gradients_fc proto:716-790, */
/* in the serial order of misc.h:119-129 (b, then j*T + t, then i).          */
/* ------------------------------------------------------------------------ */
static inline float prod_value(const float *x1, const float *x2, const float *pe, int64_t n1,
                               int64_t n2, int sliced, int32_t id, int *source, int64_t *index)
{
    if (sliced) {
        const int c = id % 3;
        const int64_t k = id / 3;
        *source = c;
        *index = k;
        return c == 0 ? x1[k] : (c == 1 ? x2[k] : pe[k]);
    }
    if (id < n1) { *source = 0; *index = id; return x1[id]; }
    if (id < n1 + n2) { *source = 1; *index = id - n1; return x2[id - n1]; }
    *source = 2;
    *index = id - n1 - n2;
    return pe[id - n1 - n2];
}

typedef struct {
    int32_t idx, alt;
    float md;
    int src1, src2;
    int64_t k1, k2;
} prod_pair;

/* lookup index, and the min-margin anchor of calculate_product_lookup_index_backprop:
 * strict |delta| < |min| from FLT_MAX (the first of equal margins wins) */
static prod_pair prod_lookup(const float *x1, const float *x2, const float *pe,
                             const int32_t *anc, int64_t n_anchors, int64_t n1, int64_t n2,
                             int sliced, float cmp_eps)
{
    prod_pair p;
    p.idx = 0; p.alt = 0; p.md = 3.402823466e+38f; p.src1 = -1; p.src2 = -1; p.k1 = 0; p.k2 = 0;
    int32_t flip = -1;
    for (int64_t k = 0; k < n_anchors; k++) {
        const int32_t a1 = anc[2 * k], a2 = anc[2 * k + 1];
        if (a1 < 0 || a2 < 0) continue; /* unused pair */
        int s1, s2;
        int64_t i1, i2;
        const float v1 = prod_value(x1, x2, pe, n1, n2, sliced, a1, &s1, &i1);
        const float v2 = prod_value(x1, x2, pe, n1, n2, sliced, a2, &s2, &i2);
        const float d = v1 - v2;
        if (rounded_greater0(d, cmp_eps)) p.idx |= (1 << k);
        if (fabsf(d) < fabsf(p.md)) {
            p.md = d; flip = (int32_t)k; p.src1 = s1; p.src2 = s2; p.k1 = i1; p.k2 = i2;
        }
    }
    p.alt = flip >= 0 ? (p.idx ^ (1 << flip)) : p.idx;
    return p;
}

/* The fp64 mode of the product oracle (a test tolerance aid, not a
 * restatement): every term the reference adds -- the weight payload row[c],
 * the pushes (float)du and -(float)du, the gradient term (float)(g*lr) -- is
 * summed in fp64 into *_sum, and its magnitude into *_abs.  Any fp32 summation
 * order of n such terms lies within n * 2^-24 * abs of sum.  NULL = off. */
typedef struct {
    double *x1_sum, *x1_abs, *x2_sum, *x2_abs, *pe_sum, *pe_abs, *w_sum, *w_abs;
} prod_acc64;

static inline void acc64_add(double *sum, double *abs_, int64_t i, double v)
{
    sum[i] += v;
    abs_[i] += fabs(v);
}

/* syn_offsets / syn_targets: sparse lookup connectivity (CSR of synapses per
 * lookup neuron, weights per synapse), or NULL for fully connected tables. */
static void fill_outputs_product_core(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    const int64_t *syn_offsets, const int32_t *syn_targets,
    int64_t batch, int64_t seq_len, int64_t n1, int64_t n2, int64_t pd, int64_t n_detectors,
    int64_t n_anchors, int64_t n_outputs, int sliced, float cmp_eps, int int_mode,
    double int_rescaler, float *out, double *out_sum, double *out_abs)
{
    const int64_t E = (int64_t)1 << n_anchors;
    for (int64_t b = 0; b < batch; b++)
        for (int64_t j = 0; j < seq_len; j++)
            for (int64_t t = 0; t < n_detectors; t++)
                for (int64_t i = 0; i < j; i++) {
                    const float *pet = pd > 0 ? pe + ((j - i - 1) * n_detectors + t) * pd : NULL;
                    const prod_pair p = prod_lookup(x1 + (b * seq_len + i) * n1, x2 + (b * seq_len + j) * n2,
                                                    pet, anchors + t * n_anchors * 2, n_anchors, n1, n2,
                                                    sliced, cmp_eps);
                    const int64_t n = t * E + p.idx;
                    const int64_t o0 = (b * seq_len + j) * n_outputs;
                    const int64_t c0 = syn_offsets ? syn_offsets[n] : 0;
                    const int64_t c1 = syn_offsets ? syn_offsets[n + 1] : n_outputs;
                    for (int64_t c = c0; c < c1; c++) {
                        /* synapse c of the neuron, or output c of the table row */
                        const int64_t o = syn_targets ? syn_targets[c] : c;
                        const float wv = syn_offsets ? w[c] : w[n * n_outputs + c];
                        if (out_sum)
                            acc64_add(out_sum, out_abs, o0 + o, (double)wv);
                        else if (int_mode)
                            as_i32(out + o0)[o] = wrap_add(as_i32(out + o0)[o],
                                                           (int32_t)((double)wv * OR_DENOM32 * int_rescaler));
                        else
                            out[o0 + o] += wv;
                    }
                }
}

void oracle_fill_outputs_product(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    int64_t batch, int64_t seq_len, int64_t n1, int64_t n2, int64_t pd, int64_t n_detectors,
    int64_t n_anchors, int64_t n_outputs, int sliced, float cmp_eps, int int_mode,
    double int_rescaler, float *out)
{
    fill_outputs_product_core(x1, x2, pe, anchors, w, NULL, NULL, batch, seq_len, n1, n2, pd,
                              n_detectors, n_anchors, n_outputs, sliced, cmp_eps, int_mode,
                              int_rescaler, out, NULL, NULL);
}

/* fill_outputs_product over sparse connectivity (fill_outputs_product_sparse_logic,
 * proto:2266-2394; CPU branch fill_outputs_product_cpu_logic proto:2148-2264):
 * every synapse of the pair's neuron commits its weight to its target. */
void oracle_fill_outputs_product_sparse(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    const int64_t *syn_offsets, const int32_t *syn_targets, int64_t batch, int64_t seq_len,
    int64_t n1, int64_t n2, int64_t pd, int64_t n_detectors, int64_t n_anchors, int64_t n_outputs,
    int sliced, float cmp_eps, int int_mode, double int_rescaler, float *out, double *out_sum,
    double *out_abs)
{
    fill_outputs_product_core(x1, x2, pe, anchors, w, syn_offsets, syn_targets, batch, seq_len, n1,
                              n2, pd, n_detectors, n_anchors, n_outputs, sliced, cmp_eps, int_mode,
                              int_rescaler, out, out_sum, out_abs);
}

void oracle_fill_outputs_product64(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    int64_t batch, int64_t seq_len, int64_t n1, int64_t n2, int64_t pd, int64_t n_detectors,
    int64_t n_anchors, int64_t n_outputs, int sliced, float cmp_eps, double *out_sum,
    double *out_abs)
{
    fill_outputs_product_core(x1, x2, pe, anchors, w, NULL, NULL, batch, seq_len, n1, n2, pd,
                              n_detectors, n_anchors, n_outputs, sliced, cmp_eps, 0, 1.0, NULL,
                              out_sum, out_abs);
}

static inline void prod_push(float *dst, double du, int int_mode, double int_rescaler)
{
    if (int_mode)
        *as_i32(dst) = wrap_add(*as_i32(dst), (int32_t)(du * OR_DENOM32 * int_rescaler));
    else
        *dst += (float)du;
}

static void propagate_product_core(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    const int64_t *syn_offsets, const int32_t *syn_targets, const float *g, int64_t batch, int64_t seq_len, int64_t n1, int64_t n2, int64_t pd,
    int64_t n_detectors, int64_t n_anchors, int64_t n_outputs, int sliced, float cmp_eps,
    double lr, int int_mode, double int_rescaler, float *x1_grad, float *x2_grad, float *pe_grad,
    float *w_grad, const prod_acc64 *acc)
{
    const int64_t E = (int64_t)1 << n_anchors;
    for (int64_t b = 0; b < batch; b++)
        for (int64_t j = 0; j < seq_len; j++)
            for (int64_t t = 0; t < n_detectors; t++)
                for (int64_t i = 0; i < j; i++) {
                    const int64_t pe_off = ((j - i - 1) * n_detectors + t) * pd;
                    const prod_pair p = prod_lookup(x1 + (b * seq_len + i) * n1, x2 + (b * seq_len + j) * n2,
                                                    pd > 0 ? pe + pe_off : NULL, anchors + t * n_anchors * 2,
                                                    n_anchors, n1, n2, sliced, cmp_eps);
                    const float *gj = g + (b * seq_len + j) * n_outputs;
                    const int64_t nm = t * E + p.idx, na = t * E + p.alt;
                    if (p.src1 >= 0) {
                        double ms = 0.0, as = 0.0;
                        if (syn_offsets) {
                            /* every synapse of the neuron, in list order (proto:2452-2489) */
                            for (int64_t c = syn_offsets[nm]; c < syn_offsets[nm + 1]; c++)
                                ms += (double)w[c] * (double)gj[syn_targets[c]];
                            for (int64_t c = syn_offsets[na]; c < syn_offsets[na + 1]; c++)
                                as += (double)w[c] * (double)gj[syn_targets[c]];
                        } else {
                            const float *rm = w + nm * n_outputs;
                            const float *ra = w + na * n_outputs;
                            for (int64_t c = 0; c < n_outputs; c++) ms += (double)rm[c] * (double)gj[c];
                            for (int64_t c = 0; c < n_outputs; c++) as += (double)ra[c] * (double)gj[c];
                        }
                        const double du = du_of_margin(p.md) * (ms - as);
                        if (fabs(du) > OR_EPS) {
                            const int64_t base[3] = {(b * seq_len + i) * n1, (b * seq_len + j) * n2, pe_off};
                            if (acc) {
                                double *sums[3] = {acc->x1_sum, acc->x2_sum, acc->pe_sum};
                                double *abss[3] = {acc->x1_abs, acc->x2_abs, acc->pe_abs};
                                if (sums[p.src1]) acc64_add(sums[p.src1], abss[p.src1], base[p.src1] + p.k1, (double)(float)du);
                                if (sums[p.src2]) acc64_add(sums[p.src2], abss[p.src2], base[p.src2] + p.k2, (double)(float)-du);
                            } else {
                                float *dst[3] = {x1_grad, x2_grad, pe_grad};
                                if (dst[p.src1]) prod_push(dst[p.src1] + base[p.src1] + p.k1, du, int_mode, int_rescaler);
                                if (dst[p.src2]) prod_push(dst[p.src2] + base[p.src2] + p.k2, -du, int_mode, int_rescaler);
                            }
                        }
                    }
                    if (acc ? acc->w_sum != NULL : w_grad != NULL) {
                        /* row nm's outputs; sparse: every synapse of neuron nm */
                        const int64_t c0 = syn_offsets ? syn_offsets[nm] : nm * n_outputs;
                        const int64_t c1 = syn_offsets ? syn_offsets[nm + 1] : (nm + 1) * n_outputs;
                        for (int64_t c = c0; c < c1; c++) {
                            const double gg = (double)gj[syn_targets ? syn_targets[c] : c - c0];
                            if (!(fabs(gg) > OR_EPS)) continue;
                            if (acc)
                                acc64_add(acc->w_sum, acc->w_abs, c, (double)(float)(gg * lr));
                            else if (int_mode)
                                as_i32(w_grad)[c] = wrap_add(as_i32(w_grad)[c], (int32_t)(gg * lr * OR_DENOM32 * int_rescaler));
                            else
                                w_grad[c] += (float)(gg * lr);
                        }
                    }
                }
}

/* x1_grad / x2_grad may alias (the layer passes one x and one x_grad twice);
 * w_grad may be NULL (Internal policy: no weight gradient in this pass). */
void oracle_propagate_product(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    const float *g, int64_t batch, int64_t seq_len, int64_t n1, int64_t n2, int64_t pd,
    int64_t n_detectors, int64_t n_anchors, int64_t n_outputs, int sliced, float cmp_eps,
    double lr, int int_mode, double int_rescaler, float *x1_grad, float *x2_grad, float *pe_grad,
    float *w_grad)
{
    propagate_product_core(x1, x2, pe, anchors, w, NULL, NULL, g, batch, seq_len, n1, n2, pd,
                           n_detectors, n_anchors, n_outputs, sliced, cmp_eps, lr, int_mode,
                           int_rescaler, x1_grad, x2_grad, pe_grad, w_grad, NULL);
}

/* oracle_propagate_product over sparse connectivity (propagate_backward_product_cpu_logic,
 * proto:2396-2628): the main and flipped sums run over every synapse of the
 * two neurons, one du per pair.  The weight gradient adds to every synapse of
 * the pair's neuron (as the GPU kernel gather_w_gradients_product_sparse,
 * proto:2946-3073, over all forward groups; the CPU branch passes output block
 * 0 and so reaches only a neuron's first group, proto:2580-2596). */
void oracle_propagate_product_sparse(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    const int64_t *syn_offsets, const int32_t *syn_targets, const float *g, int64_t batch,
    int64_t seq_len, int64_t n1, int64_t n2, int64_t pd, int64_t n_detectors, int64_t n_anchors,
    int64_t n_outputs, int sliced, float cmp_eps, double lr, int int_mode, double int_rescaler,
    float *x1_grad, float *x2_grad, float *pe_grad, float *w_grad)
{
    propagate_product_core(x1, x2, pe, anchors, w, syn_offsets, syn_targets, g, batch, seq_len, n1,
                           n2, pd, n_detectors, n_anchors, n_outputs, sliced, cmp_eps, lr, int_mode,
                           int_rescaler, x1_grad, x2_grad, pe_grad, w_grad, NULL);
}

void oracle_propagate_product_sparse64(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    const int64_t *syn_offsets, const int32_t *syn_targets, const float *g, int64_t batch,
    int64_t seq_len, int64_t n1, int64_t n2, int64_t pd, int64_t n_detectors, int64_t n_anchors,
    int64_t n_outputs, int sliced, float cmp_eps, double lr, double *x1_sum, double *x1_abs,
    double *x2_sum, double *x2_abs, double *pe_sum, double *pe_abs, double *w_sum, double *w_abs)
{
    const prod_acc64 acc = {x1_sum, x1_abs, x2_sum, x2_abs, pe_sum, pe_abs, w_sum, w_abs};
    propagate_product_core(x1, x2, pe, anchors, w, syn_offsets, syn_targets, g, batch, seq_len, n1,
                           n2, pd, n_detectors, n_anchors, n_outputs, sliced, cmp_eps, lr, 0, 1.0,
                           NULL, NULL, NULL, NULL, &acc);
}

/* fp64 mode of oracle_propagate_product (see prod_acc64); any pair of
 * sum/abs pointers may be NULL, and x1_* / x2_* may alias. */
void oracle_propagate_product64(
    const float *x1, const float *x2, const float *pe, const int32_t *anchors, const float *w,
    const float *g, int64_t batch, int64_t seq_len, int64_t n1, int64_t n2, int64_t pd,
    int64_t n_detectors, int64_t n_anchors, int64_t n_outputs, int sliced, float cmp_eps,
    double lr, double *x1_sum, double *x1_abs, double *x2_sum, double *x2_abs, double *pe_sum,
    double *pe_abs, double *w_sum, double *w_abs)
{
    const prod_acc64 acc = {x1_sum, x1_abs, x2_sum, x2_abs, pe_sum, pe_abs, w_sum, w_abs};
    propagate_product_core(x1, x2, pe, anchors, w, NULL, NULL, g, batch, seq_len, n1, n2, pd,
                           n_detectors, n_anchors, n_outputs, sliced, cmp_eps, lr, 0, 1.0, NULL,
                           NULL, NULL, NULL, &acc);
}
