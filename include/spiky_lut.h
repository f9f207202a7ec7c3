/*
 * spiky_lut.h -- C ABI of the MI355X-native LUT-layer hot path.
 *
 * One opaque manager object stands for one reference `LUTDataManagerF` /
 * `LUTDataManagerI` (spiky_cuda/lut/lut.cu:16-128, pybind at lut.cu:1476-1656).
 * The caller (Python via ctypes, or any FFI) owns every tensor: weights,
 * anchors, activations and gradients are plain device pointers, sizes are
 * plain integers, streams are `hipStream_t` passed as `void *`.  Nothing in
 * these signatures depends on torch.
 *
 * Conventions (all as in the reference):
 *   - weights  : fp32 [n_detectors * 2^n_anchors][n_outputs]   (row = t*E + idx)
 *   - anchors  : int32 pairs [n_detectors][n_anchors][2]; -1 marks an unused pair
 *   - input    : fp32 [batch][n_inputs];  output fp32 [batch][n_outputs]
 *   - idx / min_deltas / min_delta_indices : [batch][n_detectors]
 *   - outputs, input gradients and weight gradients are ACCUMULATED INTO, so
 *     callers pass zeroed buffers (reference LUTLayer.py:631,851,864).  Entry
 *     points with an `overwrite_*` flag may instead be told the buffer holds
 *     garbage and is to be written, which skips the zero-fill pass.
 *   - int32 summation managers keep partial sums as int32 fixed point
 *     (DENOMINATOR32 = 0xFFFFF scaled by int_rescaler) inside the fp32 buffers
 *     and convert back to fp32 before returning (lut_runtime_kernels_logic.proto:200-213).
 *
 * Return codes: SPIKY_OK, SPIKY_VALUE_ERROR (the reference raises ValueError),
 * SPIKY_RUNTIME_ERROR (RuntimeError: HIP failures, bad device state).  The
 * message of the last failure on the calling thread is spiky_lut_last_error().
 */
#ifndef SPIKY_LUT_H
#define SPIKY_LUT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPIKY_OK 0
#define SPIKY_VALUE_ERROR 1
#define SPIKY_RUNTIME_ERROR 2

typedef struct spiky_lut_manager spiky_lut_manager;

/* Message of the last failed call on this thread ("" if none). */
const char *spiky_lut_last_error(void);

/* Library version string. */
const char *spiky_lut_version(void);

/* Replaces LUTDataManagerF/I::LUTDataManagerF/I (lut.cu:16-128; validation
 * lut.cu:47-76).  summation_int32 != 0 gives the LUTDataManagerI behaviour
 * with the given int_rescaler (aux/lut_I.cu:1-2). */
int spiky_lut_create(uint32_t n_inputs, uint32_t n_outputs, uint32_t n_detectors,
                     uint32_t n_anchors_per_detector, uint32_t sequence_length,
                     uint32_t positional_dim, uint64_t initial_synapse_capacity,
                     uint32_t forward_group_size, uint32_t backward_group_size,
                     int summation_int32, double int_rescaler, spiky_lut_manager **out);

/* fp32 summation order of the fully connected forward (no reference
 * counterpart; default 0).  ordered != 0: one fp32 commit per block of
 * backward_group_size tables, added in ascending block order -- the reference
 * CPU path's arithmetic (lut_runtime_kernels_logic.proto:1214-1299 run serially),
 * bit for bit.  ordered == 0: at large batches the table-major forward sums
 * several blocks in fp64 before one fp32 commit, which is at least as close to
 * the exact sum and within the reference GPU path's own order-dependent fp32
 * tolerance (it commits blocks with atomics in any order).  int32 summation is
 * bit-exact either way. */
int spiky_lut_set_ordered_sums(spiky_lut_manager *m, int ordered);

/* Replaces the pybind destructor (lut.cu ~LUTDataManager). */
void spiky_lut_destroy(spiky_lut_manager *m);

/* Replaces register_synapse_meta (lut.cu:148-206). */
int spiky_lut_register_synapse_meta(spiky_lut_manager *m, float learning_rate,
                                    float min_synaptic_weight, float max_synaptic_weight,
                                    float initial_noise_level, float initial_weight,
                                    uint32_t *out_meta_index);

/* Replaces initialize_neurons (lut.cu:208-243). */
int spiky_lut_initialize_neurons(spiky_lut_manager *m, int is_fully_connected);

/* Replaces get_number_of_lookup_neurons / get_weights_dimension /
 * get_max_forward_groups_per_neuron / get_number_of_synapses
 * (lut.cu:266-301). */
uint64_t spiky_lut_n_lookup_neurons(const spiky_lut_manager *m);
uint64_t spiky_lut_weights_dimension(const spiky_lut_manager *m);
uint32_t spiky_lut_max_forward_groups_per_neuron(const spiky_lut_manager *m);
uint64_t spiky_lut_n_synapses(const spiky_lut_manager *m);

/* Replaces forward_step (lut.cu:629-716 -> lut_runtime.cu:76-211):
 * check_detectors(_eval) then fill_outputs_non_seq_{fc,sparse}.
 * min_deltas == NULL selects eval mode (lut_runtime.cu:104). */
int spiky_lut_forward_step(spiky_lut_manager *m, const float *weights, uint32_t batch_size,
                           const float *input, const int32_t *anchors, float *output,
                           int32_t *lookup_indices, float cmp_eps, float *min_deltas,
                           int32_t *min_delta_indices, void *stream);

/* Allocation-free forward.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * semantics and results as spiky_lut_forward_step, on fully connected
 * managers only; it calls no hipMalloc / hipFree.  Where the table-major
 * forward needs scratch (transposed indices and block partials), that
 * scratch is a library-owned static device array of
 * SPIKY_NOALLOC_SCRATCH_BYTES, one copy per device, held until the process
 * ends; shapes that need more return SPIKY_VALUE_ERROR without launching.
 * Every call on one device shares that device's array.  Eager calls are
 * chained on the device: each waits (hipStreamWaitEvent, on the caller's
 * stream) for the previous call's last kernel, whatever its stream, thread or
 * manager.  Calls captured into a HIP graph are not chained this way: graphs
 * replayed so that they overlap on one device race on the array. */
#define SPIKY_NOALLOC_SCRATCH_BYTES (64ull << 20)
int spiky_lut_forward_step_noalloc(spiky_lut_manager *m, const float *weights,
                                   uint32_t batch_size, const float *input, const int32_t *anchors,
                                   float *output, int32_t *lookup_indices, float cmp_eps,
                                   float *min_deltas, int32_t *min_delta_indices, void *stream);

/* int8 tables with a per-detector fp32 scale, forward (eval or train).
 * Weight of row entry = scales[t] * (float)q8[...] in fp32.  Fully connected
 * managers only.  The int8 form has no counterpart in the reference (its
 * tables are fp32, lut.h:55); it reuses forward_step's index and summation
 * semantics (lut_runtime.cu:76-211) on the dequantised weight. */
int spiky_lut_forward_step_i8(spiky_lut_manager *m, const int8_t *q8, const float *scales,
                              uint32_t batch_size, const float *input, const int32_t *anchors,
                              float *output, int32_t *lookup_indices, float cmp_eps,
                              float *min_deltas, int32_t *min_delta_indices, void *stream);

/* Replaces backward_backprop (lut.cu:1030-1088 -> lut_runtime.cu:213-397):
 * propagate_through_detectors_non_seq_* into input_grad and
 * gather_w_gradients_non_seq_* into weight_grad.  external_lr >= 0 selects the
 * Internal policy: the weight update -lr*external_lr*g is applied to `weights`
 * in place and weight_grad must be NULL (lut_runtime.cu:236-238).
 * overwrite_weight_grad != 0 tells the library weight_grad holds garbage to be
 * overwritten (no reference counterpart: it fuses the caller's zeros_like,
 * LUTLayer.py:864, into the gradient kernel). */
int spiky_lut_backward_backprop(spiky_lut_manager *m, float *weights, uint32_t batch_size,
                                const float *output_grad, const int32_t *anchors,
                                const int32_t *lookup_indices, const float *min_deltas,
                                const int32_t *min_delta_indices, float *input_grad,
                                double external_lr, float *weight_grad,
                                int overwrite_weight_grad, void *stream);

/* Replaces forward_step_concat (lut.cu pybind 1556-1575 -> lut_runtime.cu:399-593):
 * check_detectors_seq(_eval) over the batch_size*S rows of input [B][S][I],
 * check_positional_embeddings(_eval) over positional_embeddings [(S-1)][T][Npe]
 * (unused when positional_dim == 0), then fill_outputs_fully_connected_seq into
 * output [B][S][O].  Lookup indices / min deltas / min indices are [B][S][T];
 * positional ones [(S-1)][T].  min_deltas == NULL selects eval mode, and then
 * the three min-delta arguments must all be NULL.  Managers with
 * sequence_length > 1; a sparse manager runs fill_outputs_sparse_seq
 * (proto:1906-2015) over its compiled connectivity, weights per synapse. */
int spiky_lut_forward_step_concat(spiky_lut_manager *m, const float *weights, uint32_t batch_size,
                                  const float *input, const int32_t *anchors, float *output,
                                  int32_t *lookup_indices, float cmp_eps,
                                  const float *positional_embeddings,
                                  int32_t *positional_lookup_indices, float *min_deltas,
                                  int32_t *min_delta_indices, float *positional_min_deltas,
                                  int32_t *positional_min_delta_indices, void *stream);

/* Replaces backward_backprop_concat (lut.cu pybind 1620-1636 ->
 * lut_runtime.cu:595-850): propagate_through_detectors_seq_fc into input_grad
 * [B][S][I] and positional_grad [(S-1)][T][Npe], and gather_w_gradients_seq_fc
 * into weight_grad (external_lr < 0) or, for the Internal policy
 * (external_lr >= 0, weight_grad NULL), the in-place update of weights.
 * overwrite_weight_grad as for spiky_lut_backward_backprop.  A sparse manager
 * runs propagate_through_detectors_seq_sparse and gather_w_gradients_seq_sparse
 * (proto:3371-3627, 3837-3942); its weight gradient is per synapse. */
int spiky_lut_backward_backprop_concat(spiky_lut_manager *m, float *weights, uint32_t batch_size,
                                       const float *output_grad, const int32_t *anchors,
                                       const int32_t *lookup_indices, const float *min_deltas,
                                       const int32_t *min_delta_indices, float *input_grad,
                                       double external_lr, const int32_t *positional_lookup_indices,
                                       const float *positional_min_deltas,
                                       const int32_t *positional_min_delta_indices,
                                       float *positional_grad, float *weight_grad,
                                       int overwrite_weight_grad, void *stream);

/* Replaces forward_step_product (lut.cu:847-943 -> lut_runtime.cu:852-1049).  The manager is built with sequence_length 1 and
 * n_inputs = n_inputs_1 + n_inputs_2 + positional_dim; sequence_length is the
 * real one.  Every pair i < j of a sequence looks up each table over the
 * virtual row [input_1[i] | input_2[j] | pe[(j-i-1)*T + t]] (sliced_mode:
 * interleaved, virtual id = 3 * k + source).  output [B*S*O] is summed into
 * (int32 summation: the caller zeroes it; it is converted to float here).
 * positional_embeddings [(S-1)*T*pd] when positional_dim > 0.  Anchor ids
 * beyond the virtual row are skipped like unused (-1) ones.  A sparse manager
 * runs fill_outputs_product_sparse (proto:2266-2394) over its connectivity. */
int spiky_lut_forward_step_product(spiky_lut_manager *m, const float *weights, uint32_t batch_size,
                                   uint32_t sequence_length, const float *input_1,
                                   const float *input_2, const int32_t *anchors, float *output,
                                   uint32_t n_inputs_1, uint32_t n_inputs_2, int sliced_mode,
                                   float cmp_eps, const float *positional_embeddings, void *stream);

/* Replaces backward_backprop_product (lut.cu:945-1039 -> lut_runtime.cu:
 * 1051-1456).  input_grad_1/2 [B*S*n] may be the same buffer (the layer passes
 * one x twice).  external_lr >= 0 (GradientType.Internal) updates the weights
 * in place with lr * -external_lr and needs weight_grad == NULL; otherwise
 * weight_grad [T*E*O] is summed into with lr.  positional_grad [(S-1)*T*pd]
 * when positional_dim > 0.  int32 summation converts every buffer it summed
 * into to float at the end (lut_runtime.cu:1405-1456). */
int spiky_lut_backward_backprop_product(spiky_lut_manager *m, float *weights, uint32_t batch_size,
                                        uint32_t sequence_length, const float *input_1,
                                        const float *input_2, const int32_t *anchors,
                                        const float *output_grad, float *input_grad_1,
                                        float *input_grad_2, double external_lr,
                                        uint32_t n_inputs_1, uint32_t n_inputs_2, int sliced_mode,
                                        float cmp_eps, float *weight_grad,
                                        const float *positional_embeddings, float *positional_grad,
                                        void *stream);

/* Replaces add_lookup_connections + compile for sparse managers
 * (lut.cu:560-627) with this build's CSR: lookup neuron n owns synapses
 * [syn_offsets[n], syn_offsets[n+1]) whose targets are output indices in
 * syn_targets.  Host pointers; the library keeps a device copy.  The weight
 * tensor of a sparse manager has one fp32 per synapse in the same order. */
int spiky_lut_set_sparse_connectivity(spiky_lut_manager *m, const int64_t *syn_offsets,
                                      const int32_t *syn_targets, uint64_t n_synapses);

/* Replaces prepare_detectors_compact (lut_compile_time_kernels_logic.proto:70-125)
 * over a CSR of each detector's ascending input list.  Host pointers.
 * Returns SPIKY_VALUE_ERROR ("Some detectors have <= 1 input synapses",
 * lut.cu:537-550) if a detector has fewer than two inputs. */
int spiky_lut_decode_anchors_compact(const uint32_t *encoded_pairs, uint32_t n_detectors,
                                     uint32_t max_pairs_per_detector, uint32_t n_anchors,
                                     const int64_t *in_offsets, const int32_t *in_ids,
                                     int32_t *anchors_out);

/* Receptive-field index builder: replaces the reference's spatial growth
 * engine for one GrowthCommand with probability p (synapse_growth.py:11-55,
 * synapse_growth_kernels_logic.proto:69-374; inclusion test in fp32 at
 * proto:229-256).  Host pointers.  Sources are visited in ascending id order;
 * out_offsets[i]..out_offsets[i+1] delimit the ascending target ids of the
 * i-th source in that order.  Call once with out_targets == NULL to get
 * *out_total, then again with capacity >= *out_total.  cuboid = x1,y1,z1,x2,y2,z2
 * relative to the source.  max_per_source == 0 means unbounded. */
int spiky_grow_cuboid(uint32_t n_src, const int32_t *src_ids, const float *src_xyz,
                      uint32_t n_tgt, const int32_t *tgt_ids, const float *tgt_xyz,
                      const float *cuboid, float p, uint64_t seed, uint32_t max_per_source,
                      int64_t *out_offsets, int32_t *out_targets, uint64_t capacity,
                      uint64_t *out_total);

/* Replaces get_profiling_stats / reset_profiler (lut.cu:1274-1290):
 * per-operation call counts and host wall-clock (stream-ordered calls are
 * timed only up to launch, since nothing here synchronises). */
int spiky_lut_profiling_stats(const spiky_lut_manager *m, char *buf, uint64_t buf_len);
void spiky_lut_reset_profiler(spiky_lut_manager *m);

/* GPU-side timing of every launch with HIP events recorded on the launch
 * stream (no reference counterpart: the reference's profiler times on the host
 * after a device-wide synchronisation, misc.h:170-194).  While enabled, each
 * kernel family's launches are bracketed by events; spiky_lut_kernel_times
 * waits for the recorded events and writes one line "name count total_ms" per
 * family (reset != 0 clears the totals). */
int spiky_lut_set_kernel_timing(spiky_lut_manager *m, int enable);
int spiky_lut_kernel_times(spiky_lut_manager *m, char *buf, uint64_t buf_len, int reset);

/* Scratch sizing, computed on the host without touching a device (no
 * reference counterpart: the reference allocates its buffers per call).  For
 * the entry point named by `op` on this manager and batch, *needed gets the
 * bytes of device scratch that entry point grows its buffer to -- the
 * layouts its launchers lay out -- and every launcher's layout is checked
 * against its region of a buffer of `capacity` bytes (UINT64_MAX: no limit);
 * a layout that does not fit returns SPIKY_VALUE_ERROR naming the launcher
 * and the bytes it needs.  The entry points themselves refuse such a layout
 * before launching anything.  sequence_length, n_inputs_1, n_inputs_2 and
 * sliced_mode are read by the product-mode codes only. */
#define SPIKY_OP_FORWARD 0           /* spiky_lut_forward_step (and _noalloc) */
#define SPIKY_OP_FORWARD_I8 1        /* spiky_lut_forward_step_i8 */
#define SPIKY_OP_BACKWARD 2          /* spiky_lut_backward_backprop, weight gradient or Internal update */
#define SPIKY_OP_BACKWARD_NO_WGRAD 3 /* spiky_lut_backward_backprop without a weight gradient */
#define SPIKY_OP_FORWARD_CONCAT 4    /* spiky_lut_forward_step_concat */
#define SPIKY_OP_BACKWARD_CONCAT 5   /* spiky_lut_backward_backprop_concat */
#define SPIKY_OP_FORWARD_PRODUCT 6   /* spiky_lut_forward_step_product */
#define SPIKY_OP_BACKWARD_PRODUCT 7  /* spiky_lut_backward_backprop_product */
int spiky_lut_scratch_plan(spiky_lut_manager *m, int op, uint32_t batch_size, uint32_t sequence_length,
                           uint32_t n_inputs_1, uint32_t n_inputs_2, int sliced_mode, uint64_t capacity,
                           uint64_t *needed);

/* ---- dense -> sparse converter --------------------------------------------
 * Replaces DenseToSparseConverterNative (spiky_cuda/torch_utils/torch_utils.cu:
 * 11-339; Python side spiky/util/torch_utils.py:7-125).  A 32-bit word of the
 * source is kept when its bit pattern is non-zero (the reference's int4
 * compare, torch_utils_kernels_logic.proto:20-35).  Unlike the reference,
 * whose blocks claim output ranges with an atomic, the output is in ascending
 * index order.  The workspace is caller memory of
 * spiky_densify32_workspace_bytes(n) bytes on the source's device. */

/* Bytes of workspace for a source of n words. */
uint64_t spiky_densify32_workspace_bytes(uint64_t n);

/* DenseToSparseConverterNative::count_nonzero: *counter (device int64) =
 * number of non-zero words; n % 4 == 0 or SPIKY_VALUE_ERROR with the
 * reference's text.  Leaves the per-tile offsets in the workspace. */
int spiky_count_nonzero32(const void *source, uint64_t n, void *workspace,
                          uint64_t workspace_bytes, int64_t *counter, void *stream);

/* DenseToSparseConverterNative::dense_to_sparse_32: writes the indices (int64)
 * and raw 32-bit values of the non-zero words, at most `capacity` of them;
 * *counter = the number of non-zero words (which may exceed capacity: the
 * caller checks).  erase_input != 0 zeroes the kept words of the source.
 * counted != 0 reuses the workspace of an spiky_count_nonzero32 call on the
 * same, unchanged source (skips one read of it). */
int spiky_dense_to_sparse32(void *source, uint64_t n, int64_t *indices, void *values,
                            uint64_t capacity, void *workspace, uint64_t workspace_bytes,
                            int64_t *counter, int erase_input, int counted, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SPIKY_LUT_H */
