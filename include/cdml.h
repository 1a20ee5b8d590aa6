/*
 * cdml.h -- C ABI of libcdml_hip.so, the MI355X (gfx950) implementation of
 * CallaghanDev.ML's causal multi-head attention forward path.
 *
 * The library is the native half of a HIP-backed IAccelerationManager: the
 * host side (a C# manager via P/Invoke, or the C++ HipAccelerationManager in
 * callaghandev.ml_amd/host/) owns every device buffer, stream and pinned
 * staging buffer and passes plain pointers and sizes here.  The library
 * never frees a caller buffer and never allocates device memory inside a
 * kernel entry point.
 *
 * Conventions
 *   - Matrices are row-major float32 (C# float[,] layout).  A matrix
 *     argument is (pointer, rows, cols, ld) with ld >= cols the row stride
 *     in elements.  Weights are [out, in]; y = x W^T + b.
 *   - Head h of a [rows, D] activation owns columns [h*d_h, (h+1)*d_h).
 *   - Masks are uint8 [Lq, Lk], 1 = attend (bool[,] true = attend).
 *   - Kernel entry points only enqueue work on `stream` (NULL = the null
 *     stream) and return; only *_synchronize and cdml_event_elapsed_ms block.
 *   - Every function returns a status; CDML_OK is 0.  On failure
 *     cdml_last_error() returns a message for the calling thread.
 *   - Calls on distinct streams from distinct threads are safe.  One stream
 *     is not re-entrant.
 *
 * Reference paths below are relative to CallaghanDev.ML/ in the reference
 * repository.
 */
#ifndef CDML_H
#define CDML_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CDML_OK 0
#define CDML_E_INVALID (-1)  /* bad shape, null pointer, bad option         */
#define CDML_E_NODEVICE (-2) /* no usable HIP device                        */
#define CDML_E_HIP (-3)      /* a HIP runtime call failed (text in message) */
#define CDML_E_CAUSAL (-4)   /* causal attention with Lq != Lk              */

/* FFN activations, numbered as Enums/ActivationType.cs:7-15. */
#define CDML_ACT_NONE 0
#define CDML_ACT_SIGMOID 1
#define CDML_ACT_TANH 2
#define CDML_ACT_RELU 3
#define CDML_ACT_LEAKYRELU 4
#define CDML_ACT_SWISH 5
/* Or'ed into cdml_linear_backward_act's activation: dz holds the output y of
 * a cdml_linear_preact call made without z (ReLU or leaky ReLU only). */
#define CDML_ACT_FROM_OUTPUT 0x100

typedef struct cdml_stream_opaque *cdml_stream; /* a hipStream_t */
typedef struct cdml_event_opaque *cdml_event;   /* a hipEvent_t  */

typedef struct cdml_device_info {
  char name[128];
  char arch[64];         /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int compute_units;
  int max_clock_mhz;     /* shader clock used for the fp32 MFMA roofline */
  int memory_clock_mhz;
  int memory_bus_bits;
  size_t total_memory;
  size_t lds_per_workgroup;
} cdml_device_info;

/* ---- device, errors ----------------------------------------------------
 * Replaces the device set-up of AccelerationManagers/GPU/AccelerationGPU.cs:85-147
 * (ILGPU Context/Accelerator creation).  The device is process-wide; a
 * manager instance only owns streams and buffers. */
int cdml_device_count(int *count);
int cdml_init(int device);
int cdml_device_info_get(int device, cdml_device_info *info);
const char *cdml_last_error(void);
const char *cdml_version(void);

/* ---- streams and events (owned by the caller) ------------------------- */
int cdml_stream_create(cdml_stream *stream);
int cdml_stream_destroy(cdml_stream stream);
int cdml_stream_synchronize(cdml_stream stream);
/* Makes later work on `stream` wait for the work recorded before `event`
 * (on any stream), without blocking the host: a host that downloads one part
 * of a result on a copy stream while the kernel computes the next part on
 * its own stream.  No counterpart in the reference (ILGPU runs one stream). */
int cdml_stream_wait_event(cdml_stream stream, cdml_event event);
int cdml_event_create(cdml_event *event);
/* An event for host waits only (no timestamps; cdml_event_elapsed_ms
 * rejects it): lighter to record, for the per-chunk events of a staged
 * download.  No counterpart in the reference, whose ILGPU copies are
 * synchronous (TransformerCore.cs:1300-1348). */
int cdml_event_create_sync_only(cdml_event *event);
int cdml_event_destroy(cdml_event event);
int cdml_event_record(cdml_event event, cdml_stream stream);
/* Blocks until the work recorded before `event` has finished (a host that
 * stages a download in chunks copies chunk i out of pinned memory while the
 * later chunks are still in flight). */
int cdml_event_synchronize(cdml_event event);
/* Waits for `stop`, then returns the time between the two events. */
int cdml_event_elapsed_ms(cdml_event start, cdml_event stop, float *ms);

/* ---- memory (owned by the caller) --------------------------------------
 * Replace the per-call Allocate1D/CopyFromCPU/CopyToCPU/Dispose pattern of
 * AccelerationManagers/GPU/TransformerCore.cs:1300-1348. */
int cdml_malloc(void **ptr, size_t bytes);
int cdml_free(void *ptr);
int cdml_host_alloc_pinned(void **ptr, size_t bytes);
int cdml_host_free_pinned(void *ptr);
int cdml_memcpy_h2d_async(void *dst, const void *src, size_t bytes, cdml_stream stream);
int cdml_memcpy_d2h_async(void *dst, const void *src, size_t bytes, cdml_stream stream);
int cdml_memcpy_d2d_async(void *dst, const void *src, size_t bytes, cdml_stream stream);
/* ---- recorded launch sequences (no counterpart in the reference, whose
 * managers launch every kernel from the host).  A caller that repeats one
 * sequence of enqueue calls on a stream (a generation loop, a training step
 * of fixed shape) records it once between cdml_graph_capture_begin and
 * cdml_graph_capture_end, then replays it with cdml_graph_launch: one host
 * call instead of one per kernel, with the recorded arguments and pointers.
 * While recording, only enqueue calls on that stream are legal (no
 * synchronisation, no copies from pageable host memory); a failed call
 * leaves the recording open, and cdml_graph_capture_end then discards it
 * (graph NULL). */
typedef struct cdml_graph_s *cdml_graph;
int cdml_graph_capture_begin(cdml_stream stream);
int cdml_graph_capture_end(cdml_stream stream, cdml_graph *graph);
int cdml_graph_launch(cdml_graph graph, cdml_stream stream);
int cdml_graph_destroy(cdml_graph graph);

/* Zero `count` floats with a fill kernel (safe under stream capture). */
int cdml_zero_f32_async(float *dst, size_t count, cdml_stream stream);
/* dst[i] = value for i < count, a fill kernel (safe under stream capture). */
int cdml_fill_i32_async(int *dst, size_t count, int value, cdml_stream stream);
/* Strided device copy: `height` rows of `width_bytes` bytes, row pitches in
 * bytes (used to place a [batch, len, dim] block into a [batch, t_max, dim]
 * decode cache). */
int cdml_memcpy2d_d2d_async(void *dst, size_t dpitch, const void *src,
                            size_t spitch, size_t width_bytes, size_t height,
                            cdml_stream stream);

/* ---- hot-path kernels (device pointers) -------------------------------- */

/* IAccelerationManager.ProjectQKV (IAccelerationManager.cs:169), replacing
 * AccelerationCPU.cs:2005-2069 / AccelerationMutliThreadCPU.cs:798-831 /
 * GPU/TransformerCore.cs:1386-1464,1629-1665:
 *   q = x wq^T + bq,  k = x wk^T + bk,  v = x wv^T + bv
 * x [rows, in_dim]; w* [out_dim, in_dim]; b* [out_dim] (NULL = zero bias);
 * q, k, v [rows, out_dim], contiguous.  One launch, fp32 MFMA. */
int cdml_project_qkv(const float *x, const float *wq, const float *bq,
                     const float *wk, const float *bk, const float *wv,
                     const float *bv, float *q, float *k, float *v, int rows,
                     int in_dim, int out_dim, cdml_stream stream);

/* IAccelerationManager.ProjectOutputBatch (IAccelerationManager.cs:259) and
 * BatchDotProductAddBias (:45-50) followed by ApplyActivationInPlace
 * (Neural Network/NeuralNetwork.cs:670-702), replacing
 * AccelerationCPU.cs:2694-2715 and :342-404:
 *   y = act(x w^T + b)
 * x [rows, in_dim] with row stride ldx; w [out_dim, in_dim]; b [out_dim] or
 * NULL; y [rows, out_dim] with row stride ldy; activation CDML_ACT_*. */
int cdml_linear(const float *x, int ldx, const float *w, const float *b,
                float *y, int ldy, int rows, int in_dim, int out_dim,
                int activation, cdml_stream stream);

/* IAccelerationManager.MatrixMultiply (:20), replacing AccelerationCPU.cs:
 * 159-214 (the FFN backward's hidden deltas and input gradient,
 * NeuralNetwork.cs:861-881): c = a b with a [m, k] (row stride lda), b
 * [k, n] (row stride ldb), c [m, n] (row stride ldc); fp32 MFMA.
 * MatrixMultiplyTranspose (:26, a b^T) is cdml_linear with b as the weight
 * and no bias. */
int cdml_matmul(const float *a, int lda, const float *b, int ldb, float *c,
                int ldc, int m, int k, int n, cdml_stream stream);

/* IAccelerationManager.BackpropLinearProjection (:182) and
 * BackpropOutputProjection (:184), replacing AccelerationCPU.cs:2188-2270:
 *   wgrad += dy^T x,  bgrad += column sums of dy,  dx (+)= dy w
 * x [rows, in_dim] (row stride ldx); dy [rows, out_dim] (row stride lddy);
 * w [out_dim, in_dim]; wgrad [out_dim, in_dim] and bgrad [out_dim]
 * accumulate; dx [rows, in_dim] (row stride lddx) is overwritten
 * (accumulate_dx = 0, BackpropOutputProjection) or added to (1,
 * BackpropLinearProjection).  dx = NULL skips the input gradient; wgrad and
 * bgrad may be NULL to skip theirs.  fp32 MFMA; the bias gradient is summed
 * inside the weight-gradient GEMM.  When the weight gradient has too few
 * output tiles to fill the device (rows >> in_dim * out_dim / 2^15), its
 * reduction over rows is split into chunks whose partial sums go to
 * `workspace` and are added in a fixed order (deterministic, no atomics):
 * `workspace` is 16-byte aligned device memory of at least
 * cdml_linear_backward_workspace_size() bytes (NULL when that is 0). */
int cdml_linear_backward_workspace_size(int rows, int in_dim, int out_dim,
                                        size_t *bytes);
int cdml_linear_backward(const float *x, int ldx, const float *dy, int lddy,
                         const float *w, float *dx, int lddx, float *wgrad,
                         float *bgrad, int rows, int in_dim, int out_dim,
                         int accumulate_dx, void *workspace,
                         size_t workspace_bytes, cdml_stream stream);

/* IAccelerationManager.BackpropQKV (:171), replacing AccelerationCPU.cs:
 * 2071-2186:
 *   dx = dq wq + dk wk + dv wv   (overwritten)
 *   w*_grad += d*^T x,  b*_grad += column sums of d*   (accumulated)
 * x [rows, in_dim]; dq, dk, dv [rows, out_dim]; w* and w*_grad
 * [out_dim, in_dim]; b*_grad [out_dim]; dx [rows, in_dim]; all contiguous.
 * `workspace`: split-K partials of the three weight gradients, as for
 * cdml_linear_backward, of cdml_backprop_qkv_workspace_size() bytes. */
int cdml_backprop_qkv_workspace_size(int rows, int in_dim, int out_dim,
                                     size_t *bytes);
int cdml_backprop_qkv(const float *x, const float *dq, const float *dk,
                      const float *dv, const float *wq, const float *wk,
                      const float *wv, float *wq_grad, float *bq_grad,
                      float *wk_grad, float *bk_grad, float *wv_grad,
                      float *bv_grad, float *dx, int rows, int in_dim,
                      int out_dim, void *workspace, size_t workspace_bytes,
                      cdml_stream stream);

/* IAccelerationManager.ApplyRotaryPositionEmbeddingInPlace (:320) and
 * ApplyRotaryPositionEmbeddingHeadInPlace (:319), replacing
 * AccelerationCPU.cs:4855-4980 and GPU/RotaryPositionEmbeddings.cs:58-156.
 * In place on x [rows, ld]: heads h = 0..num_heads-1 of width head_dim start
 * at column start_col + h*head_dim; pairs (2p, 2p+1) rotate by
 * theta = pos / powf(base_theta, 2p / head_dim) (sin negated when inverse).
 * Position of row r: positions[r] when `positions` (device int32[rows]) is
 * non-NULL, else pos_offset + (seg_len > 0 ? r % seg_len : r); seg_len is the
 * segmented trainer's per-sequence length (TransformerTrainer.cs:811-848),
 * positions the decode step's absolute position (LanguageModel.cs:432-480).
 * head_dim must be even and <= 512. */
int cdml_rope(float *x, int rows, int ld, int start_col, int head_dim,
              int num_heads, float base_theta, int inverse, int pos_offset,
              int seg_len, const int *positions, cdml_stream stream);

/* The rotation table of cdml_rope for positions 0..n_pos-1: cs (device,
 * 8-byte aligned, n_pos * head_dim floats) receives (cos theta, sin theta) of
 * pair p at position pos in cs[2 * (pos * head_dim/2 + p) + {0, 1}], computed
 * with cdml_rope's arithmetic.  No counterpart of its own in the reference:
 * it serves cdml_project_qkv_rope, the fusion of the ProjectQKV and
 * ApplyRotaryPositionEmbeddingInPlace calls of MultiHeadAttention.Forward
 * (MultiHeadAttention.cs:96-111). */
int cdml_rope_table(float *cs, int n_pos, int head_dim, float base_theta,
                    cdml_stream stream);

/* The trainer's ApplySegmentedRotaryInPlace(q, k, numHeads, segmentLength,
 * inverse) (TransformerTrainer.cs:811-848, the inverse at :980): heads
 * h = 0..num_heads-1 of width head_dim, from column 0 of q and of k (both
 * [rows, ld], device, different arrays; k may be NULL), rotated in place from
 * a cdml_rope_table of n_pos positions, with the same bits as cdml_rope at
 * that table's base.  Row r has position pos_offset + (seg_len > 0 ?
 * r % seg_len : r), which must be below n_pos; rows * num_heads * head_dim / 2
 * below 2^31. */
int cdml_rope_qk_table(float *q, float *k, int rows, int ld, int head_dim,
                       int num_heads, const float *rope_cs, int n_pos,
                       int pos_offset, int seg_len, int inverse,
                       cdml_stream stream);

/* cdml_project_qkv followed by the forward rotary embedding of Q and K, as
 * MultiHeadAttention.Forward calls ProjectQKV and then
 * applies the rotary embedding to Q and K (MultiHeadAttention.cs:108-110,
 * RotaryPositionEmbedding.cs:20-73), in one launch: the rotation is applied in the projection's
 * epilogue from a cdml_rope_table of n_pos positions.  Row r has position
 * pos_offset + (seg_len > 0 ? r % seg_len : r), which must be below n_pos.
 * head_dim must be even and divide out_dim; V is not rotated. */
int cdml_project_qkv_rope(const float *x, const float *wq, const float *bq,
                          const float *wk, const float *bk, const float *wv,
                          const float *bv, float *q, float *k, float *v,
                          int rows, int in_dim, int out_dim, int head_dim,
                          const float *rope_cs, int n_pos, int pos_offset,
                          int seg_len, cdml_stream stream);

/* IAccelerationManager.ScaledDotProductAttention (:167) and
 * MultiHeadAttentionForward (:155), replacing AccelerationCPU.cs:1797-1956
 * and :1647-1792 and GPU/TransformerCore.cs:659-834,1142-1349.
 * Fused flash-style forward over `batch` independent sequences:
 *   q [batch, lq, ldq], k [batch, lk, ldk], v [batch, lk, ldv],
 *   o [batch, lq, ldo]; dim = num_heads * head_dim columns are used.
 * For each sequence, head and query i: keys j < (causal ? i+1 : lk) with
 * mask[i*lk + j] != 0 (mask NULL = all) get weight softmax(q.k * scale);
 * a row with no such key is written as 0.  ScaledDotProductAttention passes
 * scale = 1/sqrtf(head_dim) (AccelerationCPU.cs:1865).  causal requires
 * lq == lk (CDML_E_CAUSAL otherwise, AccelerationCPU.cs:1859-1862). */
int cdml_sdpa_fwd(const float *q, int ldq, const float *k, int ldk,
                  const float *v, int ldv, float *o, int ldo, int batch,
                  int lq, int lk, int dim, int num_heads, float scale,
                  int causal, const uint8_t *mask, cdml_stream stream);

/* cdml_sdpa_fwd that also keeps each row's softmax statistics for a later
 * cdml_sdpa_bwd_saved: lse (device, [batch * num_heads][lq] floats, an
 * opaque per-row normaliser).  Head dims up to 128. */
int cdml_sdpa_fwd_lse(const float *q, int ldq, const float *k, int ldk,
                      const float *v, int ldv, float *o, int ldo, float *lse,
                      int batch, int lq, int lk, int dim, int num_heads,
                      float scale, int causal, const uint8_t *mask,
                      cdml_stream stream);

/* MultiHeadAttention.Forward (self-attention, MultiHeadAttention.cs:96-111
 * and AttentionCore :146-155) for one layer on device buffers: ProjectQKV,
 * the rotary embedding of Q and K, ScaledDotProductAttention (scale
 * 1/sqrt(head_dim), causal or masked) and ProjectOutputBatch, as one call:
 *   x [batch * seq_len, dim] -> y [batch * seq_len, dim]
 * for `batch` sequences of seq_len rows (row r at position r % seq_len).
 * Weights [dim, dim] as the reference stores them, biases [dim] or NULL.
 * rope_cs: a cdml_rope_table of at least seq_len positions, or NULL to build
 * one (base rope_base) in the workspace.  workspace: 256-byte aligned, at
 * least cdml_mha_layer_fwd_workspace_size bytes (Q, K, V and the attention
 * output, each rows * dim floats, and the table).  The same results as the
 * three entries cdml_project_qkv_rope, cdml_sdpa_fwd and cdml_linear. */
int cdml_mha_layer_fwd_workspace_size(int batch, int seq_len, int dim,
                                      int num_heads, size_t *bytes);
int cdml_mha_layer_fwd(const float *x, const float *wq, const float *bq,
                       const float *wk, const float *bk, const float *wv,
                       const float *bv, const float *wo, const float *bo,
                       float *y, int batch, int seq_len, int dim,
                       int num_heads, float rope_base, int causal,
                       const uint8_t *mask, const float *rope_cs,
                       void *workspace, size_t workspace_bytes,
                       cdml_stream stream);

/* IAccelerationManager.MultiHeadAttentionBackward, both overloads (:161,
 * :163), replacing AccelerationCPU.cs:1011-1280.  For `batch` independent
 * sequences (the segmented trainer's SegmentedMultiHeadAttentionBackward,
 * TransformerTrainer.cs:989-1060, is batch = segment count):
 *   q, dout [batch, lq, ld*]; k, v [batch, lk, ld*]; dq [batch, lq, lddq];
 *   dk, dv [batch, lk, ld*]; all three gradients are overwritten.
 * Visible keys of query i: j <= i when causal (the useDecoderMask overload;
 * lq may differ from lk), and mask[i*lk + j] != 0 when mask is non-NULL
 * (the bool[,] overload).  scale is used as passed (the attention scores are
 * q.k * scale).  A query with no visible key contributes nothing.
 * `workspace`: device memory of cdml_sdpa_bwd_workspace_size() bytes.  Head
 * dims up to 128 run on fp32 MFMA (a forward pass with row statistics, then
 * dK/dV and dQ kernels, no atomics; head dims other than 32, 64 and 128, and
 * rows that are not 16-byte aligned, take zero-padded scalar loads); larger
 * head dims run a per-row kernel. */
int cdml_sdpa_bwd_workspace_size(int batch, int lq, int lk, int dim,
                                 int num_heads, size_t *bytes);
/* A larger workspace for cdml_sdpa_bwd: the required bytes plus room for the
 * dS blocks, 2 * lq^2 bytes per (sequence, head), when the shape can use them
 * (causal without a mask, lq == lk, head dim 32 or 64, 16-byte aligned rows).
 * With it the dK/dV pass stores dS and dQ is one product over it instead of
 * recomputing the scores; the result meets the same bar but need not match
 * the smaller workspace's bits.  Other shapes leave the extra bytes unused. */
int cdml_sdpa_bwd_stored_ds_workspace_size(int batch, int lq, int lk, int dim,
                                           int num_heads, int causal,
                                           size_t *bytes);
int cdml_sdpa_bwd(const float *q, int ldq, const float *k, int ldk,
                  const float *v, int ldv, const float *dout, int lddo,
                  float *dq, int lddq, float *dk, int lddk, float *dv,
                  int lddv, int batch, int lq, int lk, int dim, int num_heads,
                  float scale, int causal, const uint8_t *mask,
                  void *workspace, size_t workspace_bytes, cdml_stream stream);

/* cdml_sdpa_bwd from the forward pass's own output o (row stride ldo) and
 * row statistics lse, as cdml_sdpa_fwd_lse wrote them for the same q, k, v,
 * scale, causal flag and mask: no forward pass is repeated.  This is the
 * trainer's form (TransformerTrainer keeps the attention output in its
 * cache, AttentionCache.cs:9-38).  Head dims up to 128; workspace: at least
 * batch * num_heads * lq floats.  With cdml_sdpa_bwd_saved_workspace_size()
 * bytes (causal without a mask, lq == lk, head dim 32 or 64, 16-byte aligned
 * rows) the dK/dV pass also stores dS, 2 * lq^2 bytes per (sequence, head),
 * and dQ becomes one product over it instead of recomputing the scores; the
 * result meets the same bar but need not match the smaller workspace's bits. */
int cdml_sdpa_bwd_saved_workspace_size(int batch, int lq, int lk, int dim,
                                       int num_heads, int causal,
                                       size_t *bytes);
int cdml_sdpa_bwd_saved(const float *q, int ldq, const float *k, int ldk,
                        const float *v, int ldv, const float *o, int ldo,
                        const float *lse, const float *dout, int lddo,
                        float *dq, int lddq, float *dk, int lddk, float *dv,
                        int lddv, int batch, int lq, int lk, int dim,
                        int num_heads, float scale, int causal,
                        const uint8_t *mask, void *workspace,
                        size_t workspace_bytes, cdml_stream stream);

/* cdml_sdpa_bwd_saved followed by the inverse rotary embedding of dQ and dK,
 * as TransformerTrainer.BackpropAttention applies it to the attention's
 * input gradients (TransformerTrainer.cs:978-985, the inverse of the rotation
 * at :811-848): every head of a row at the row's index within its sequence
 * (dQ rows modulo lq, dK rows modulo lk), with rope_cs a cdml_rope_table of
 * n_pos >= max(lq, lk) positions for the head dim (8-byte aligned).  dK, and
 * dQ where it is recomputed, are rotated as the kernels store them; dQ from
 * stored dS blocks takes one table-RoPE launch on dQ alone.  With lq == lk
 * (the trainer's causal self-attention) the bits are those of
 * cdml_sdpa_bwd_saved then cdml_rope_qk_table(dq, dk, ..., pos_offset 0,
 * seg_len lq, inverse 1) on the same rows.  Same workspace as
 * cdml_sdpa_bwd_saved; the head dim must be even. */
int cdml_sdpa_bwd_saved_rope(const float *q, int ldq, const float *k, int ldk,
                             const float *v, int ldv, const float *o, int ldo,
                             const float *lse, const float *dout, int lddo,
                             float *dq, int lddq, float *dk, int lddk,
                             float *dv, int lddv, int batch, int lq, int lk,
                             int dim, int num_heads, float scale, int causal,
                             const uint8_t *mask, const float *rope_cs,
                             int n_pos, void *workspace,
                             size_t workspace_bytes, cdml_stream stream);

/* ---- training step (TransformerTrainer.TrainBatchDiscrete,
 * Transformers/MultiTypeTransformer/TransformerTrainer.cs:217-327) -------- */

/* IAccelerationManager.FFNForwardBatch's layer with its cache, the forward
 * pass that NeuralNetwork.ComputeInputGradientBatch recomputes
 * (Neural Network/NeuralNetwork.cs:824-839): z = x w^T + b and y = act(z),
 * both [rows, out_dim] with row stride ldy.  With ReLU or leaky ReLU, z may
 * be NULL: y alone then carries the derivative (CDML_ACT_FROM_OUTPUT), ReLU
 * writing its zero as -0 where z < 0 or z is NaN (the reference's
 * derivative is 1 at z >= 0, 0 elsewhere); leaky ReLU's y has the sign of z.
 * The values equal y = act(z) as numbers. */
int cdml_linear_preact(const float *x, int ldx, const float *w, const float *b,
                       float *z, float *y, int ldy, int rows, int in_dim,
                       int out_dim, int activation, cdml_stream stream);

/* One layer of NeuralNetwork.ComputeInputGradientBatch (NeuralNetwork.cs:
 * 841-881) on fp32 MFMA, with cdml_linear_backward's gradients:
 *   wgrad += dy^T x,  bgrad += column sums of dy,
 *   dx = (dy w) * act'(dz) + add
 * dz (the layer below's pre-activation, for its hidden deltas) and add (a
 * residual gradient, MatrixAddInPlace) may be NULL; both have row stride
 * lddx.  act' follows FillActivationAndDerivative (NeuralNetwork.cs:885-944).
 * activation | CDML_ACT_FROM_OUTPUT: dz is instead the output y of a
 * cdml_linear_preact call made without z, and act' comes from it with the
 * same values.  workspace as cdml_linear_backward. */
int cdml_linear_backward_act(const float *x, int ldx, const float *dy,
                             int lddy, const float *w, const float *dz,
                             int activation, const float *add, float *dx,
                             int lddx, float *wgrad, float *bgrad, int rows,
                             int in_dim, int out_dim, void *workspace,
                             size_t workspace_bytes, cdml_stream stream);

/* IAccelerationManager.ResidualLayerNormForward (:140), replacing
 * AccelerationCPU.cs:1440-1514: out = gamma * normalized + beta with
 * residual = a + b, per-row mean and biased variance, normalized =
 * (residual - mean) / sqrt(variance + eps).  mean / variance [rows],
 * residual / normalized [rows, features] are written when non-NULL.
 * features <= 2048. */
int cdml_residual_layernorm_fwd(const float *a, const float *b,
                                const float *gamma, const float *beta,
                                float *out, float *mean, float *variance,
                                float *residual, float *normalized, int rows,
                                int features, float eps, cdml_stream stream);

/* IAccelerationManager.LayerNormBackward (:143), replacing AccelerationCPU.cs:
 * 1516-1564.  The upstream gradient is dout + dout2 (dout2 NULL: dout alone;
 * the two gradients of a residual branch).  normalized may be NULL: it is
 * then recomputed from input (the residual), mean and variance with the
 * forward's arithmetic.  dinput [rows, features] is written; dgamma / dbeta
 * [features] are written, or added to (accumulate = 1, the trainer's
 * VectorAccumulate), or skipped when NULL.  Column sums run in a fixed
 * order through `workspace` (cdml_layernorm_backward_workspace_size bytes).
 * features <= 2048. */
int cdml_layernorm_backward_workspace_size(int rows, int features,
                                           size_t *bytes);
int cdml_layernorm_backward(const float *dout, const float *dout2,
                            const float *normalized, const float *gamma,
                            const float *input, const float *mean,
                            const float *variance, float *dinput,
                            float *dgamma, float *dbeta, int rows,
                            int features, float eps, int accumulate,
                            void *workspace, size_t workspace_bytes,
                            cdml_stream stream);

/* IAccelerationManager.CrossEntropyLossAndGradient (:207-209), replacing
 * AccelerationCPU.cs:2377-2440: for rows i < effective_len with target
 * targets[i] (device int32, in [0, out_dim)): p = softmax(logits[i]),
 * dlogits[i] = (p - onehot) / effective_len * grad_scale; rows past
 * effective_len get 0.  *loss (device float) = mean over those rows of
 * -log(p[target] + 1e-10), times loss_scale.  grad_scale is the trainer's
 * per-bucket ScaleMatrixLocal (TransformerTrainer.cs:291-294).  A target
 * outside [0, out_dim) makes the loss NaN.  workspace:
 * cdml_cross_entropy_workspace_size bytes. */
int cdml_cross_entropy_workspace_size(int rows, size_t *bytes);
int cdml_cross_entropy(const float *logits, int ldl, const int *targets,
                       int rows, int out_dim, int effective_len,
                       float grad_scale, float loss_scale, float *loss,
                       float *dlogits, int lddl, void *workspace,
                       size_t workspace_bytes, cdml_stream stream);

/* IAccelerationManager.MSELossAndGradient (:212-214), replacing
 * AccelerationCPU.cs:2442-2490: rows i < effective_len of pred [rows,
 * out_dim] against targets rows i (row strides ldp / ldt): dout = 2 (p - t) /
 * (effective_len * out_dim) * grad_scale, *loss (device) = mean squared
 * difference times loss_scale; rows past effective_len get 0.  workspace:
 * rows floats. */
int cdml_mse_loss(const float *pred, int ldp, const float *targets, int ldt,
                  int rows, int out_dim, int effective_len, float grad_scale,
                  float loss_scale, float *loss, float *dout, int ldd,
                  void *workspace, size_t workspace_bytes, cdml_stream stream);

/* IAccelerationManager.MatrixAddInPlace (:91; AccelerationCPU.cs:
 * 522-546): target[i] += addend[i] for `count` floats. */
int cdml_add_inplace(float *target, const float *addend, size_t count,
                     cdml_stream stream);

/* IAccelerationManager.MatrixUpdate / VectorUpdate (:246, :248), replacing
 * AccelerationCPU.cs:2548-2597: weights[i] -= learning_rate * gradients[i]
 * (product and difference rounded separately) for `count` floats. */
int cdml_update_f32(float *weights, const float *gradients,
                    float learning_rate, size_t count, cdml_stream stream);

/* IAccelerationManager.MatrixScaleInPlace / VectorScaleInPlace (:235, :240),
 * replacing AccelerationCPU.cs:2514-2546: x[i] *= scale. */
int cdml_scale_f32(float *x, float scale, size_t count, cdml_stream stream);

/* IAccelerationManager.MatrixSquaredNorm / VectorSquaredNorm (:221, :226),
 * replacing AccelerationCPU.cs:2493-2512: out[0] (device) = sum of x[i]^2,
 * in a fixed order (512 block partials, then their sum).  workspace:
 * cdml_sum_squares_workspace_size bytes. */
int cdml_sum_squares_workspace_size(size_t *bytes);
int cdml_sum_squares(const float *x, size_t count, float *out, void *workspace,
                     size_t workspace_bytes, cdml_stream stream);

/* IAccelerationManager.AccumulateTokenEmbeddingGrad (:203-205), replacing
 * AccelerationCPU.cs:2339-2370, as a gather over groups of rows that share a
 * token: for group k, rows order[group_start[k] .. group_start[k+1]) of
 * dx (+ dx2, both row stride ldx) are added in that order to row
 * group_token[k] of grad [vocab, dim].  With rows listed in increasing
 * order this is the reference's summation order, and no two groups share a
 * token, so no atomics are needed.  All index arrays are device int32. */
int cdml_embedding_grad(float *grad, const float *dx, const float *dx2,
                        int ldx, const int *order, const int *group_start,
                        const int *group_token, int n_groups, int dim,
                        cdml_stream stream);

/* One parameter tensor of the update: weight and grad are device arrays of
 * `count` floats.  Consecutive entries with equal `group` are summed
 * together before being added to the global squared norm (the trainer adds
 * WQ + WK + WV + WO as one term). */
typedef struct cdml_param {
  float *weight;
  float *grad;
  long long count;
  int group;
  int reserved;
} cdml_param;

/* ScaleGradients + ComputeGradientNorm + ClipGradients
 * (TransformerTrainer.cs:1306-1384, MatrixSquaredNorm AccelerationCPU.cs:
 * 2493-2512): params is a device array of `count` entries.  Norm of the
 * gradients scaled by `prescale` (1 / validCount); result (device float[3])
 * receives the norm, the clipping factor (threshold / norm when use_clipping
 * and norm > threshold, else 1) and 1 if the norm is finite, else 0.
 * workspace: cdml_grad_norm_workspace_size bytes. */
int cdml_grad_norm_workspace_size(int count, size_t *bytes);
int cdml_grad_norm(const cdml_param *params, int count, float prescale,
                   int use_clipping, float threshold, float *result,
                   void *workspace, size_t workspace_bytes,
                   cdml_stream stream);

/* UpdateParameters (TransformerTrainer.cs:1269-1305; MatrixUpdate /
 * VectorUpdate AccelerationCPU.cs:2548-2597): with g' = (g * prescale) *
 * clip factor (result[1] from cdml_grad_norm), w -= learning_rate * g' when
 * result[2] is nonzero.  zero_grads = 1 clears the gradients for the next
 * step (ZeroAllGradients); 0 leaves g' in them, as the reference's in-place
 * scaling does. */
int cdml_sgd_update(const cdml_param *params, int count, float learning_rate,
                    float prescale, const float *result, int zero_grads,
                    cdml_stream stream);

/* Single-query decode attention over a cached K/V, the device form of the
 * inline loop in LanguageModel.DecoderSelfAttentionStep
 * (Transformers/MultiTypeTransformer/LanguageModel.cs:365-427), which has no
 * IAccelerationManager slot in the reference.
 *   q [batch, dim]; kcache, vcache [batch, t_max, dim]; kv_len device
 *   int32[batch] (keys [0, kv_len[b]) are attended, 0 <= kv_len <= t_max);
 *   o [batch, dim].
 * Split-K over the cache with a combine pass; `workspace` is caller-owned
 * device memory of at least cdml_decode_attn_workspace_size() bytes. */
int cdml_decode_attn_workspace_size(int batch, int t_max, int dim,
                                    int num_heads, size_t *bytes);
int cdml_decode_attn(const float *q, const float *kcache, const float *vcache,
                     const int *kv_len, float *o, int batch, int t_max,
                     int dim, int num_heads, float scale, void *workspace,
                     size_t workspace_bytes, cdml_stream stream);

/* cdml_decode_attn without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split-K partials live in a static device array of the library, one per
 * GPU, of CDML_DECODE_NOALLOC_MAX_BYTES; shapes whose partials
 * (cdml_decode_attn_workspace_size) exceed it fail with CDML_E_INVALID.
 * Allocates nothing and frees nothing.  Every call on one GPU shares that
 * array: calls that overlap on one GPU (two streams, two threads) race, so
 * such callers must order them.  Results are identical to cdml_decode_attn's
 * (same kernels). */
#define CDML_DECODE_NOALLOC_MAX_BYTES (32u << 20)
int cdml_decode_attn_noalloc(const float *q, const float *kcache,
                             const float *vcache, const int *kv_len, float *o,
                             int batch, int t_max, int dim, int num_heads,
                             float scale, cdml_stream stream);

/* Appends one K row and one V row per sequence to the decode cache, as
 * LanguageModel.cs:356-363 does: kcache[b, positions[b], :] = k_new[b, :]
 * (same for V).  positions is device int32[batch], each in [0, t_max). */
int cdml_kv_cache_append(const float *k_new, const float *v_new,
                         float *kcache, float *vcache, const int *positions,
                         int batch, int t_max, int dim, cdml_stream stream);

/* IAccelerationManager.ResidualLayerNorm (:132), replacing
 * AccelerationCPU.cs:1376-1438: y = gamma * (s - mean) / sqrt(var + eps) + beta
 * with s = a + b per row, biased variance.  a, b, y [rows, features]. */
int cdml_residual_layernorm(const float *a, const float *b, const float *gamma,
                            const float *beta, float *y, int rows,
                            int features, float eps, cdml_stream stream);

/* IAccelerationManager.EmbedTokenIds (:275-277), replacing
 * AccelerationCPU.cs:3473-3515: out[i, :] = table[ids[i], :].  ids is device
 * int32[count]; an id outside [0, vocab) writes a zero row and, when
 * bad_count (device int32) is non-NULL, increments it. */
int cdml_embed_tokens(const int *ids, int count, const float *table, int vocab,
                      int dim, float *out, int *bad_count, cdml_stream stream);

/* Greedy next-token choice over logits x [rows, cols] (row stride ld):
 * out[i * out_stride] = the lowest column index holding the row maximum
 * (NaN entries never win).  The reference always samples
 * (LanguageModel.SampleFromLogits, LanguageModel.cs:551-584); this is the
 * deterministic argmax the greedy-generation parity checks use, kept on the
 * device so a generation loop needs no host round trip per token. */
int cdml_argmax_rows(const float *x, int rows, int cols, int ld, int *out,
                     int out_stride, cdml_stream stream);

/* ---- whole greedy decode steps of a small decoder-only model in one launch.
 * LanguageModel.Generate's per-token loop (LanguageModel.cs:482-537) runs
 * DecoderSelfAttentionStep (:334-430) in every post-LN block
 * (TransformerBlock.cs:35-44), then the LM head and the token choice.  For a
 * model of D <= 256 that is two dozen launches of microseconds each per
 * token; here one workgroup per sequence runs every step in one launch.
 *
 * Step s = 1 .. n_steps feeds token tokens[(s - 1) * batch + b] of sequence
 * b at position pos0 + s - 1. It goes through every layer:
 *   - Q/K/V with RoPE from rope_cs (as cdml_rope_table writes it);
 *   - K and V appended as row pos0 + s - 1 of the layer's caches
 *     ([batch, max_seq, dim]);
 *   - attention over the pos0 + s keys so far, scale 1 / sqrt(dim / heads);
 *   - output projection, residual LayerNorm (eps), the FFN layers, residual
 *     LayerNorm.
 * The LM head's argmax (lowest index on ties, 0 when every logit is NaN,
 * as cdml_argmax_rows) goes to tokens[s * batch + b].
 *
 * Limits: dim <= 256 with a head dim that is a multiple of 4, FFN widths
 * <= 1024 and multiples of 4, heads * max_seq <= 4096, pos0 + n_steps <=
 * max_seq; every weight row 16-byte aligned.  `layers` is a device array of
 * n_layers descriptors; every pointer in it is device memory, and each layer
 * is first checked with cdml_tiny_layer_check on the host copy.  No
 * counterpart in the reference's interface: it is the device engine's
 * generation loop. */
#define CDML_TINY_MAX_FF 4
typedef struct {
  const float *wq, *bq, *wk, *bk, *wv, *bv, *wo, *bo;  /* [dim, dim], [dim] */
  const float *ln1g, *ln1b, *ln2g, *ln2b;              /* [dim] */
  const float *ffw[CDML_TINY_MAX_FF];  /* [ffrows[f], ffcols[f]] */
  const float *ffb[CDML_TINY_MAX_FF];  /* [ffrows[f]] */
  int ffrows[CDML_TINY_MAX_FF], ffcols[CDML_TINY_MAX_FF], ffact[CDML_TINY_MAX_FF];
  int n_ff;
  float *kcache, *vcache;  /* [batch capacity, max_seq, dim] */
} cdml_tiny_layer;
typedef struct {
  const float *embedding;      /* [vocab, dim] */
  const float *out_w, *out_b;  /* [vocab, dim], [vocab] */
  const float *rope_cs;        /* [max_seq, dim / heads / 2] (cos, sin) pairs */
  const cdml_tiny_layer *layers;
  int n_layers, dim, heads, vocab, max_seq;
  float eps;
} cdml_tiny_model;
int cdml_tiny_layer_check(const cdml_tiny_layer *layer, int dim);
int cdml_tiny_decode(const cdml_tiny_model *model, int *tokens, int batch,
                     int pos0, int n_steps, cdml_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* CDML_H */
