// lut_kernels.h -- launchers of the LUT hot-path kernels (gfx950 / CDNA4).
//
// Internal to libspiky_lut.so; the public C ABI is include/spiky_lut.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

namespace spiky {

// ---- scratch ---------------------------------------------------------------
// Device memory beyond a launcher's inputs and outputs (partials, keys,
// buckets) comes in a caller-owned buffer described by a Scratch.  A launcher
// lays its regions out with a ScratchLayout before it launches anything, so
// the bytes it asks for and the bytes it addresses come from one layout:
//   Plan  -- record the layout's end in `needed`, launch nothing;
//   Check -- also refuse a layout that ends past `bytes`, launch nothing;
//   Run   -- refuse such a layout (hipErrorInvalidValue, nothing launched),
//            else launch.
// In Plan and Check modes no pointer argument is read: they may be null.
struct Scratch {
    enum Mode { Plan, Check, Run };
    void *ptr = nullptr;
    size_t bytes = 0;
    Mode mode = Run;
    size_t needed = 0;  // set by the launcher
};

inline Scratch scratch_plan() {
    Scratch s;
    s.mode = Scratch::Plan;
    return s;
}

inline Scratch scratch_run(void *ptr, size_t bytes) {
    Scratch s;
    s.ptr = ptr;
    s.bytes = bytes;
    return s;
}

// Why the last launcher on this thread refused its scratch (empty if none).
inline std::string &scratch_refusal() {
    thread_local std::string why;
    return why;
}

class ScratchLayout {
  public:
    explicit ScratchLayout(Scratch &s) : s_(s) {}
    // The next region: n bytes at a 256-byte boundary.
    template <typename T>
    T *take(size_t n) {
        off_ = (off_ + 255) & ~(size_t)255;
        T *p = reinterpret_cast<T *>(reinterpret_cast<uintptr_t>(s_.ptr) + off_);
        off_ += n;
        return p;
    }
    size_t end() const { return off_; }
    // After the last take(): true when the launcher returns *err now, without
    // launching (Plan or Check mode, or a layout past the buffer's end).
    bool stop(hipError_t *err, const char *who) {
        s_.needed = off_;
        *err = hipSuccess;
        if (s_.mode != Scratch::Plan && off_ > s_.bytes) {
            scratch_refusal() = std::string(who) + ": its scratch layout needs " + std::to_string(off_) +
                                " bytes, " + std::to_string(s_.bytes) + " given";
            *err = hipErrorInvalidValue;
            return true;
        }
        return s_.mode != Scratch::Run;
    }

  private:
    Scratch &s_;
    size_t off_ = 0;
};

// spiky_cuda/misc/misc.h:90 (EPS) and misc.h:98-99 (DENOMINATOR32 and its reciprocal)
constexpr double kEps = 0.00000000000000001;
constexpr double kDenom32 = 1048575.0;
constexpr double kDenom32Reciproc = 9.536752259018191e-07;

struct FcShape {
    uint32_t batch;
    uint32_t n_inputs;
    uint32_t n_outputs;
    uint32_t n_detectors;
    uint32_t n_anchors;
    uint32_t n_entries;  // 2^n_anchors
    uint32_t dgs;        // detectors per fp64 partial sum (backward_group_size)
    uint32_t ogs;        // outputs per gradient dot block (forward_group_size)
    // fp32 summation: true keeps one fp32 commit per block of dgs tables in
    // ascending block order (bit-identical to the reference CPU path); false lets
    // the table-major forward sum several blocks in fp64 before one commit
    bool ordered_sums = false;
};

// check_detectors(_eval): lookup index, and in train mode the min-margin anchor.
hipError_t launch_check_detectors(const FcShape &s, const float *x, const int32_t *anchors,
                                  float cmp_eps, int32_t *idx, float *min_deltas,
                                  int32_t *min_idx, hipStream_t st);

// Row gather-sum over fp32 tables (int_mode: int32 fixed-point accumulation).
hipError_t launch_fill_fc_f32(const FcShape &s, const float *w, const int32_t *idx, float *out,
                              bool int_mode, double int_rescaler, hipStream_t st);

// Row gather-sum over int8 tables with a per-detector fp32 scale.
hipError_t launch_fill_fc_i8(const FcShape &s, const int8_t *q8, const float *scales,
                             const int32_t *idx, float *out, bool int_mode, double int_rescaler,
                             hipStream_t st);

// Min-margin input gradient.
hipError_t launch_propagate_fc(const FcShape &s, const float *w, const float *g,
                               const int32_t *idx, const float *min_deltas,
                               const int32_t *min_idx, const int32_t *anchors, float *x_grad,
                               bool int_mode, double int_rescaler, hipStream_t st);

// Table-row gradient: target[row, o] += lr * g[b, o] for every sample b hitting row.
// The bucketed path lays out its buckets and commit values in scratch (none for
// the atomic fallback).  key_t, when given, holds the transposed keys
// [T][key_pitch] (lookup index << key_shift in the low 16 bits) that
// launch_propagate_tm leaves at the start of its scratch.
hipError_t launch_wgrad_fc(const FcShape &s, const float *g, const int32_t *idx, float *target,
                           double lr, bool int_mode, double int_rescaler, bool overwrite,
                           Scratch &scratch, hipStream_t st, const uint32_t *key_t = nullptr,
                           uint32_t key_pitch = 0, uint32_t key_shift = 7);

// int32 fixed point -> fp32, in place.
hipError_t launch_convert_i2f(float *buf, uint64_t n, double int_rescaler, hipStream_t st);

// Stable counting sort of samples by lookup index (one wavefront per table):
// offsets [n_detectors][E+1], samples [n_detectors][batch].
hipError_t launch_bucket_samples(const FcShape &s, const int32_t *idx, int32_t *offsets,
                                 int32_t *samples, hipStream_t st,
                                 const uint32_t *key_t = nullptr, uint32_t key_pitch = 0,
                                 uint32_t key_shift = 7);

// ---- table-major fully connected path (lut_tm.hip) ------------------------
// Forward gather-sum through per-unit partials in scratch.  With
// s.ordered_sums (and always for int32 summation) it is bit-identical to
// launch_fill_fc_f32; otherwise each partial is the fp64 sum of several
// blocks, committed in ascending order.  Applies to fp32 tables with E <= 256
// and O % 4 == 0.
bool tm_fill_applies(const FcShape &s, bool int_mode);
hipError_t launch_fill_tm(const FcShape &s, const float *w, const int32_t *idx, float *out,
                          bool int_mode, double int_rescaler, Scratch &scratch, hipStream_t st);
// The same with int8 tables and one fp32 scale per table (weight = scale * q).
hipError_t launch_fill_tm_i8(const FcShape &s, const int8_t *q8, const float *scales,
                             const int32_t *idx, float *out, bool int_mode, double int_rescaler,
                             Scratch &scratch, hipStream_t st);

// fp32-summation min-margin input gradient through per-slice partial dots.
// out[i] (+)= sum over k of part[k][i] in ascending k (fp32, or wrapping int32
// then the int epilogue), i < n, n % 4 == 0.
hipError_t launch_block_commit(const uint32_t *part, float *out, uint64_t n, uint32_t n_blocks,
                               bool int_mode, double int_rescaler, hipStream_t st);
bool tm_propagate_applies(const FcShape &s);
// Row pitch (samples) and row shift of the transposed keys the table-major
// propagate writes.
uint32_t tm_key_pitch(uint32_t batch);
uint32_t tm_key_row_shift(const FcShape &s);
hipError_t launch_propagate_tm(const FcShape &s, const float *w, const float *g,
                               const int32_t *idx, const float *min_deltas,
                               const int32_t *min_idx, const int32_t *anchors, float *x_grad,
                               Scratch &scratch, hipStream_t st);

// Commit values of the weight gradient for every (row, output) of g
// (lut_fc.hip k_wgrad_commit_values).
hipError_t launch_wgrad_commit_values(const float *g, uint32_t *cv, uint64_t n, double lr,
                                      bool int_mode, double int_rescaler, hipStream_t st);

// ---- sequence-concat path (lut_seq.hip) ------------------------------------
struct SeqShape {
    uint32_t batch;
    uint32_t seq;          // sequence length S (> 1)
    uint32_t n_inputs;
    uint32_t n_outputs;
    uint32_t n_detectors;
    uint32_t n_anchors;
    uint32_t pe_dim;       // positional_dim (0: no positional embedding)
    uint32_t dgs;
    uint32_t ogs;
};
// check_detectors_seq(_eval) + check_positional_embeddings(_eval) +
// fill_outputs_fully_connected_seq; md == null selects eval mode.
hipError_t launch_forward_seq(const SeqShape &s, const float *w, const float *x,
                              const int32_t *anchors, const float *pe, float *out, int32_t *idx,
                              int32_t *pidx, float *md, int32_t *mi, float *pmd, int32_t *pmi,
                              float cmp_eps, bool int_mode, double int_rescaler, Scratch &scratch,
                              hipStream_t st);
// propagate_through_detectors_seq_fc + gather_w_gradients_seq_fc; target is the
// weight gradient (or the weights for the Internal policy, lr folded in), or null.
hipError_t launch_backward_seq(const SeqShape &s, float *w, const float *g, const int32_t *anchors,
                               const int32_t *idx, const float *md, const int32_t *mi,
                               const int32_t *pidx, const float *pmd, const int32_t *pmi,
                               float *x_grad, float *pe_grad, float *target, double lr,
                               bool overwrite, bool int_mode, double int_rescaler, Scratch &scratch,
                               hipStream_t st);

// Zero n floats with a kernel (graph-capture safe, unlike hipMemsetAsync).
hipError_t launch_zero(float *buf, uint64_t n, hipStream_t st);

// ---- sparse (CSR) path ---------------------------------------------------
// Lookup neuron n = t*E + e owns synapses [syn_offsets[n], syn_offsets[n+1]);
// syn_targets holds output indices; the weight tensor has one fp32 per synapse.
struct SparseShape {
    FcShape fc;            // n_outputs, n_detectors, n_entries ... as above
    uint32_t max_groups;   // max forward groups (of fc.ogs synapses) per lookup neuron
    bool uniform = false;  // every lookup neuron of a detector has the same synapse count
    uint32_t max_row = 0;  // most synapses of one lookup neuron
    uint32_t typ_row = 0;  // the median synapse count of the lookup neurons that have any
};

// Output-major index for the exact forward, valid when every lookup neuron of
// a detector has the same target list ("uniform" topology, ProjectionLUTLayer):
// for output j, in_pairs[in_offsets[j] .. in_offsets[j+1]) are 4-int entries
// {t, o, len, 0} in ascending (t, k): synapse k of detector t's neurons targets
// j, o = syn_offsets[t * E] + k and len the synapses a neuron of t (row e's
// synapse k is at o + e * len; total synapses below 2^31).  order[0 .. n_order)
// lists outputs by descending list length (ties in output order); fp32 sums
// may leave out the outputs with empty lists (their sums are the output's own
// value), int32 sums must list every output (the conversion rewrites it).
// With sparse_fill_by_sample(s) the launcher lays out the lookup indices
// table-major in `scr` (T * batch bytes, two a key past 256 rows); otherwise it
// takes no scratch and ignores the order.
bool sparse_fill_by_sample(const SparseShape &s);
hipError_t launch_fill_sparse_uniform(const SparseShape &s, const float *w, const int32_t *idx,
                                      const int64_t *syn_offsets, const int64_t *in_offsets,
                                      const int32_t *in_pairs, const uint32_t *order, uint32_t n_order,
                                      float *out, bool int_mode, double int_rescaler, Scratch &scr,
                                      hipStream_t st);

// Generic forward: one thread per (b, t, group), fp32 (or int32) atomics.
hipError_t launch_fill_sparse_atomic(const SparseShape &s, const float *w, const int32_t *idx,
                                     const int64_t *syn_offsets, const int32_t *syn_targets,
                                     float *out, bool int_mode, double int_rescaler,
                                     hipStream_t st);

hipError_t launch_propagate_sparse(const SparseShape &s, const float *w, const float *g,
                                   const int32_t *idx, const float *min_deltas,
                                   const int32_t *min_idx, const int32_t *anchors,
                                   const int64_t *syn_offsets, const int32_t *syn_targets,
                                   float *x_grad, bool int_mode, double int_rescaler,
                                   hipStream_t st);

// syn_neuron[s] = the lookup neuron of synapse s.  overwrite: target starts
// from zero (it is not read).  Scratch: the FC path's bucket arrays.  On a
// uniform topology row_pairs lists (t, k) int pairs, one for synapse k of each
// detector's rows (n_row_pairs = synapses / E); given, the gradient walks a
// detector's samples once per k instead of once per synapse.
hipError_t launch_wgrad_sparse(const SparseShape &s, const float *g, const int32_t *idx,
                               const int64_t *syn_offsets, const int32_t *syn_targets,
                               const int32_t *syn_neuron, const int32_t *row_pairs, uint32_t n_row_pairs,
                               float *target, double lr, bool overwrite, bool int_mode, double int_rescaler,
                               Scratch &scratch, uint64_t n_synapses, hipStream_t st);

// ---- product mode (concatenation_product == False, lut_product.hip) ---------
// Sequence-concat over sparse connectivity (lut_seq_sparse.hip).  The lookup
// indices of the B*S rows and of the distances (check_detectors_seq,
// check_positional_embeddings) come from launch_seq_indices.
hipError_t launch_seq_indices(const SeqShape &s, const float *x, const int32_t *anchors,
                              const float *pe, int32_t *idx, int32_t *pidx, float *md, int32_t *mi,
                              float *pmd, int32_t *pmi, float cmp_eps, hipStream_t st);
bool seq_sparse_applies(const SeqShape &s, uint32_t max_groups);
// out (+)= the pairs' synapse weights; int32 payloads converted at the end.
hipError_t launch_fill_seq_sparse(const SeqShape &s, uint32_t max_groups, const float *w,
                                  const int32_t *idx, const int32_t *pidx, const int64_t *syn_offsets,
                                  const int32_t *syn_targets, float *out, bool int_mode,
                                  double int_rescaler, hipStream_t st);
// Input and positional gradients, and (target != null) the synapse weight
// gradient with lr (target == w: the Internal policy, applied after the
// input gradient read the weights).
hipError_t launch_backward_seq_sparse(const SeqShape &s, uint32_t max_groups, const float *w,
                                      const float *g, const int32_t *anchors, const int32_t *idx,
                                      const float *md, const int32_t *mi, const int32_t *pidx,
                                      const float *pmd, const int32_t *pmi,
                                      const int64_t *syn_offsets, const int32_t *syn_targets,
                                      uint64_t n_synapses, float *x_grad, float *pe_grad,
                                      float *target, double lr, bool overwrite, bool int_mode,
                                      double int_rescaler, hipStream_t st);

struct ProductShape {
    uint32_t batch, seq_len, n1, n2, pd, n_detectors, n_anchors, n_outputs;
    bool sliced;
    float cmp_eps;
};
bool product_applies(const ProductShape &s);
// out (+)= sum over pairs i < j and tables of W[t][lookup]; int32 payloads
// when int_mode (the caller converts).
hipError_t launch_forward_product(const ProductShape &s, const float *w, const float *x1,
                                  const float *x2, const float *pe, const int32_t *anchors,
                                  float *out, bool int_mode, double int_rescaler, Scratch &scratch,
                                  hipStream_t st);
// Input, positional and (target != null) weight gradients; x1_grad may alias
// x2_grad.  target gets lr * g terms (weight gradient, or the weights
// themselves with lr = meta lr * -external lr for the Internal policy).
// Sparse lookup connectivity (weights per synapse of the CSR).
bool product_sparse_applies(const ProductShape &s);
hipError_t launch_forward_product_sparse(const ProductShape &s, const float *w, const float *x1,
                                         const float *x2, const float *pe, const int32_t *anchors,
                                         const int64_t *syn_offsets, const int32_t *syn_targets,
                                         float *out, bool int_mode, double int_rescaler,
                                         hipStream_t st);
hipError_t launch_backward_product_sparse(const ProductShape &s, const float *w, const float *x1,
                                          const float *x2, const float *pe, const int32_t *anchors,
                                          const int64_t *syn_offsets, const int32_t *syn_targets,
                                          const float *g, float *x1_grad, float *x2_grad,
                                          float *pe_grad, float *target, double lr, bool int_mode,
                                          double int_rescaler, hipStream_t st);
hipError_t launch_backward_product(const ProductShape &s, const float *w, const float *x1,
                                   const float *x2, const float *pe, const int32_t *anchors,
                                   const float *g, float *x1_grad, float *x2_grad, float *pe_grad,
                                   float *target, double lr, bool int_mode, double int_rescaler,
                                   Scratch &scratch, hipStream_t st);

// ---- dense -> sparse compaction of 32-bit words (lut_densify.hip) ---------
// Workspace (tile counts, then offsets) for a source of n words (n % 4 == 0).
uint64_t densify32_workspace_bytes(uint64_t n);
// Counts the non-zero words of src into the workspace and *total (device).
hipError_t launch_densify32_count(const uint32_t *src, uint64_t n, void *workspace,
                                  int64_t *total, hipStream_t st);
// After launch_densify32_count on the same src: writes the non-zero words'
// indices and values in ascending order (at most `capacity`), zeroing them in
// src when erase is set.
hipError_t launch_densify32_write(uint32_t *src, uint64_t n, const void *workspace,
                                  int64_t *indices, uint32_t *values, uint64_t capacity, bool erase,
                                  hipStream_t st);

}  // namespace spiky
