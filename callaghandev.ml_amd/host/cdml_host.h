// Host side of the MI355X attention path, above the C ABI of include/cdml.h.
//
// HipAccelerationManager mirrors the hot-path methods of the reference's
// IAccelerationManager (CallaghanDev.ML/AccelerationManagers/
// IAccelerationManager.cs): same method names, same argument meaning, same
// validation order and the same exception kinds (ArgumentNullException,
// ArgumentOutOfRangeException, ArgumentException, InvalidOperationException),
// host arrays in and host arrays out.  It is what a C# HipAccelerationManager
// does through P/Invoke: the manager owns its stream, device buffers and a
// resident copy of every weight array it has seen (identity-keyed, with a
// shadow compare, as AccelerationManagers/GPU/DeviceResidentCache.cs:44-120).
//
// MultiHeadAttention, TransformerBlock and LanguageModel restate the
// reference's Transformers/MultiTypeTransformer classes on top of the manager,
// so the reference's call sequence (ProjectQKV -> RoPE -> ScaledDotProduct-
// Attention -> ProjectOutputBatch -> ResidualLayerNorm -> FFN -> ...) runs
// unchanged against the HIP kernels.
//
// DeviceLanguageModel is the device-resident engine for the same model: all
// weights and activations stay in HBM, a whole batch of sequences runs per
// launch, prompts are prefilled in one pass, and greedy generation keeps its
// KV cache and its chosen tokens on the device.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>
#include <unordered_map>
#include <utility>
#include <vector>

#include "cdml.h"

namespace cdml_host {

// ---- exceptions named after the .NET ones the reference throws -----------
struct ArgumentException : std::invalid_argument {
  std::string param;
  explicit ArgumentException(const std::string &msg, const std::string &p = "")
      : std::invalid_argument(p.empty() ? msg : msg + " (Parameter '" + p + "')"), param(p) {}
};
struct ArgumentNullException : ArgumentException {
  explicit ArgumentNullException(const std::string &p)
      : ArgumentException("Value cannot be null.", p) {}
};
struct ArgumentOutOfRangeException : ArgumentException {
  explicit ArgumentOutOfRangeException(const std::string &p, const std::string &msg = "")
      : ArgumentException(msg.empty() ? "Specified argument was out of the range of valid values."
                                      : msg,
                          p) {}
};
struct InvalidOperationException : std::logic_error {
  explicit InvalidOperationException(const std::string &msg) : std::logic_error(msg) {}
};
struct FileNotFoundException : std::runtime_error {  // System.IO.FileNotFoundException
  explicit FileNotFoundException(const std::string &msg) : std::runtime_error(msg) {}
};

// ---- host arrays (row-major, the float[,] layout) ------------------------
// Storage of large host arrays (staging.cpp): blocks of 1 MiB and more are
// recycled through a process-wide cache (up to 1 GiB of idle blocks) instead
// of going back to the OS, so a result array of the same size as an earlier
// one lands in memory that is already mapped (a freshly mapped block costs a
// page fault per 4 KiB on its first write).  .NET's large-object heap keeps
// its segments the same way.
void *HostArrayAlloc(size_t bytes);
void HostArrayFree(void *p, size_t bytes);

// An allocator that leaves new elements uninitialised, for result arrays
// that a device download overwrites completely (their zero fill would cost a
// pass over the memory), on the recycled storage above.
template <class T>
struct DefaultInitAllocator : std::allocator<T> {
  template <class U>
  struct rebind {
    using other = DefaultInitAllocator<U>;
  };
  DefaultInitAllocator() = default;
  template <class U>
  DefaultInitAllocator(const DefaultInitAllocator<U> &) noexcept {}  // NOLINT
  T *allocate(size_t n) { return static_cast<T *>(HostArrayAlloc(n * sizeof(T))); }
  void deallocate(T *p, size_t n) noexcept { HostArrayFree(p, n * sizeof(T)); }
  template <class U>
  void construct(U *p) noexcept {
    ::new (static_cast<void *>(p)) U;
  }
  template <class U, class... A>
  void construct(U *p, A &&...args) {
    ::new (static_cast<void *>(p)) U(std::forward<A>(args)...);
  }
};
using FloatBuf = std::vector<float, DefaultInitAllocator<float>>;

struct Matrix {
  int rows = 0, cols = 0;
  FloatBuf data;
  Matrix() = default;
  Matrix(int r, int c) : rows(r), cols(c), data((size_t)r * c, 0.f) {}
  // Storage without the zero fill; every element must be written.
  static Matrix Uninit(int r, int c) {
    Matrix m;
    m.rows = r;
    m.cols = c;
    m.data.resize((size_t)r * c);
    return m;
  }
  float *ptr() { return data.data(); }
  const float *ptr() const { return data.data(); }
  float &at(int r, int c) { return data[(size_t)r * cols + c]; }
  float at(int r, int c) const { return data[(size_t)r * cols + c]; }
};

// Non-owning views; `data == nullptr` plays the role of a null reference.
struct MatView {
  const float *data = nullptr;
  int rows = 0, cols = 0;
  MatView() = default;
  MatView(const float *d, int r, int c) : data(d), rows(r), cols(c) {}
  MatView(const Matrix &m) : data(m.ptr()), rows(m.rows), cols(m.cols) {}  // NOLINT
  bool null() const { return data == nullptr; }
};
struct MatRef {
  float *data = nullptr;
  int rows = 0, cols = 0;
  MatRef() = default;
  MatRef(float *d, int r, int c) : data(d), rows(r), cols(c) {}
  MatRef(Matrix &m) : data(m.ptr()), rows(m.rows), cols(m.cols) {}  // NOLINT
};
struct VecView {
  const float *data = nullptr;
  int length = 0;
  VecView() = default;
  VecView(const float *d, int n) : data(d), length(n) {}
  VecView(const std::vector<float> &v) : data(v.data()), length((int)v.size()) {}  // NOLINT
  bool null() const { return data == nullptr; }
};
struct VecRef {  // a writable float[] (gradient accumulators)
  float *data = nullptr;
  int length = 0;
  VecRef() = default;
  VecRef(float *d, int n) : data(d), length(n) {}
  VecRef(std::vector<float> &v) : data(v.data()), length((int)v.size()) {}  // NOLINT
  bool null() const { return data == nullptr; }
};
struct MaskView {  // bool[Lq, Lk], nonzero = attend
  const uint8_t *data = nullptr;
  int rows = 0, cols = 0;
  bool null() const { return data == nullptr; }
};
struct BoolMatrix {
  int rows = 0, cols = 0;
  std::vector<uint8_t> data;
};

// FFN activations, numbered as the reference's Enums/ActivationType.cs:7-15.
enum ActivationType { None = 0, Sigmoid = 1, Tanh = 2, Relu = 3, Leakyrelu = 4, Swish = 5 };

// The transformer FFN: a NeuralNetwork with layer widths [D, FF, D] and
// activations [None, act, None] (TransformerBlock.cs:101-123).  Layer i
// (i >= 1) maps with weights[i-1] [width_i, width_{i-1}] and biases[i-1],
// then applies activations[i-1] (NeuralNetwork.cs:629-668).
struct FeedForwardNetwork {
  std::vector<Matrix> weights;
  std::vector<std::vector<float>> biases;
  std::vector<int> activations;
  int input_size() const { return weights.empty() ? 0 : weights.front().cols; }
  int output_size() const { return weights.empty() ? 0 : weights.back().rows; }
};

// ---- host copies (staging.cpp) ---------------------------------------------
// memcpy / memcmp split over a process-wide pool of host threads for large
// sizes (the pool has min(7, 3/4 of the CPUs) threads beside the caller, or
// CDML_HOST_COPY_THREADS).
void ParallelMemcpy(void *dst, const void *src, size_t bytes);
bool ParallelEqual(const void *a, const void *b, size_t bytes);
void ParallelZero(void *dst, size_t bytes);
int HostCopyThreads();

// The attention backward's workspace: the stored-dS size (the causal 32 x 32
// fp32 dS blocks, about 2 L^2 bytes per head: gigabytes at long context)
// when its extra bytes over the base size are at most `extra_cap`, else the
// base size.
size_t SdpaBackwardWorkspaceChoice(size_t base_bytes, size_t stored_ds_bytes, size_t extra_cap);
constexpr size_t kStoredDsExtraBytesCap = size_t(1) << 30;

// ---- the manager -----------------------------------------------------------
class HipAccelerationManager {
 public:
  explicit HipAccelerationManager(int device = 0);
  ~HipAccelerationManager();
  HipAccelerationManager(const HipAccelerationManager &) = delete;
  HipAccelerationManager &operator=(const HipAccelerationManager &) = delete;

  // IAccelerationManager.ProjectQKV (IAccelerationManager.cs:169)
  std::tuple<Matrix, Matrix, Matrix> ProjectQKV(MatView input, MatView WQ, VecView biasQ,
                                                MatView WK, VecView biasK, MatView WV,
                                                VecView biasV);
  // IAccelerationManager.ScaledDotProductAttention (:167)
  Matrix ScaledDotProductAttention(MatView q, MatView k, MatView v, int numHeads,
                                   MaskView mask = {}, bool causal = false);
  // IAccelerationManager.MultiHeadAttentionForward (:155)
  Matrix MultiHeadAttentionForward(MatView Q, MatView K, MatView V, int numHeads, float scale,
                                   MaskView mask = {});
  // IAccelerationManager.ProjectOutputBatch (:259)
  Matrix ProjectOutputBatch(MatView hidden, MatView outputProjection, VecView outputBias,
                            int seqLen, int outputDim);
  // IAccelerationManager.BatchDotProductAddBias (:45-50), both overloads
  Matrix BatchDotProductAddBias(MatView weights, MatView inputMatrix, VecView bias);
  Matrix BatchDotProductAddBias(MatView weights, MatView inputMatrix, int rowStart, int rowCount,
                                VecView bias);
  // IAccelerationManager.ApplyRotaryPositionEmbeddingInPlace / HeadInPlace (:319-320)
  void ApplyRotaryPositionEmbeddingInPlace(MatRef matrix, int numHeads, float baseTheta,
                                           bool inverse);
  void ApplyRotaryPositionEmbeddingHeadInPlace(MatRef matrix, int startCol, int headDim,
                                               float baseTheta, bool inverse);
  // IAccelerationManager.ResidualLayerNorm (:132)
  Matrix ResidualLayerNorm(MatView input, MatView subLayer, VecView gamma, VecView beta,
                           float epsilon = 1e-5f);
  // IAccelerationManager.EmbedTokenIds (:275-277), both overloads
  Matrix EmbedTokenIds(const std::vector<int> &tokenIds, MatView embedding, int embeddingDim);
  Matrix EmbedTokenIds(const std::vector<int> &tokenIds, int tokenStart, int tokenCount,
                       MatView embedding, int embeddingDim);
  // IAccelerationManager.CreateCausalMask (:149)
  BoolMatrix CreateCausalMask(int seqLen);
  // IAccelerationManager.FFNForwardBatch (:165) with the network the reference
  // passes as a delegate target (AccelerationCPU.cs:1957-2002 takes the
  // NeuralNetwork.ForwardPassOnlyBatch route for it).
  Matrix FFNForwardBatch(MatView input, int seqLen, int outputDim, const FeedForwardNetwork &ffn);

  // ---- attention backward (the training path of TransformerTrainer) -------
  // IAccelerationManager.MultiHeadAttentionBackward (:161, :163): gradients
  // of the attention core with respect to post-RoPE Q, K and V.  The first
  // overload is causal when useDecoderMask (keys j <= i), the second takes an
  // explicit bool[seqLenQ, seqLenK] mask (null = all keys).
  std::tuple<Matrix, Matrix, Matrix> MultiHeadAttentionBackward(MatView Q, MatView K, MatView V,
                                                                MatView dConcatenated,
                                                                int numHeads, float scale,
                                                                bool useDecoderMask = false);
  std::tuple<Matrix, Matrix, Matrix> MultiHeadAttentionBackward(MatView Q, MatView K, MatView V,
                                                                MatView dConcatenated,
                                                                int numHeads, float scale,
                                                                MaskView mask);
  // IAccelerationManager.BackpropQKV (:171): returns dInput; the weight and
  // bias gradients accumulate into the caller's arrays.
  Matrix BackpropQKV(MatView input, MatView dQ, MatView dK, MatView dV, MatView WQ, MatView WK,
                     MatView WV, MatRef WQGrad, VecRef biasQGrad, MatRef WKGrad, VecRef biasKGrad,
                     MatRef WVGrad, VecRef biasVGrad);
  // IAccelerationManager.BackpropLinearProjection (:182): weightGrad, biasGrad
  // and dInput all accumulate.
  void BackpropLinearProjection(MatView input, MatView dOutput, MatView weights, MatRef weightGrad,
                                VecRef biasGrad, MatRef dInput);
  // IAccelerationManager.BackpropOutputProjection (:184): returns dX
  // [seqLen, embeddingDim]; weightGrad and biasGrad accumulate.
  Matrix BackpropOutputProjection(MatView dLogits, MatView input, MatView weights,
                                  MatRef weightGrad, VecRef biasGrad, int seqLen, int outputDim,
                                  int embeddingDim);
  // IAccelerationManager.BackpropInputProjection (:197): weightGrad
  // [embeddingDim, inputFeatureDim] += dX^T continuousInput[inputRowStart ..
  // inputRowStart + seqLen, 0 .. inputFeatureDim), biasGrad += column sums of
  // dX.  dX is read as seqLen rows of embeddingDim floats from its start, as
  // the reference's flat span does.
  void BackpropInputProjection(MatView dX, MatView continuousInput, int inputRowStart, MatRef weightGrad,
                               VecRef biasGrad, int seqLen, int embeddingDim, int inputFeatureDim);

  // ---- the rest of the training step with real work per call ---------------
  // IAccelerationManager.MatrixMultiply (:20) / MatrixMultiplyTranspose (:26)
  Matrix MatrixMultiply(MatView A, MatView B);
  Matrix MatrixMultiplyTranspose(MatView A, MatView B);
  // IAccelerationManager.ResidualLayerNormForward (:138): (output, means,
  // variances, normalized, residual)
  std::tuple<Matrix, std::vector<float>, std::vector<float>, Matrix, Matrix>
  ResidualLayerNormForward(MatView input, MatView subLayer, VecView gamma, VecView beta,
                           float epsilon = 1e-5f);
  // IAccelerationManager.LayerNormBackward (:143): (dInput, dGamma, dBeta)
  std::tuple<Matrix, std::vector<float>, std::vector<float>>
  LayerNormBackward(MatView dOut, MatView normalized, VecView gamma, MatView input, VecView mean,
                    VecView variance, float epsilon = 1e-5f);
  // IAccelerationManager.CrossEntropyLossAndGradient (:207, :209)
  std::pair<float, Matrix> CrossEntropyLossAndGradient(MatView logits, const std::vector<int> &targets,
                                                       int targetStart, int effectiveLen);
  // IAccelerationManager.MSELossAndGradient (:212, :214)
  std::pair<float, Matrix> MSELossAndGradient(MatView predictions, MatView targets, int targetStart,
                                              int effectiveLen);
  // IAccelerationManager.AccumulateTokenEmbeddingGrad (:203, :205)
  void AccumulateTokenEmbeddingGrad(MatRef embeddingGrad, MatView dX, const std::vector<int> &tokenIds,
                                    int tokenStart, int seqLen, int embeddingDim);

  // ---- the elementwise methods the trainer calls (IAccelerationManager.cs:
  // 80-97, 221-248; AccelerationCPU.cs:507-570, 2493-2597).  The in-place
  // ones update the array's device copy and write the result back to it.
  void ZeroMatrix(MatRef matrix);
  void ZeroVector(VecRef vector);
  void MatrixAddInPlace(MatRef target, MatView addend);
  void VectorAccumulate(VecRef target, VecView source);
  float MatrixSquaredNorm(MatView matrix);
  float VectorSquaredNorm(VecView vector);
  void MatrixScaleInPlace(MatRef matrix, float scale);
  void VectorScaleInPlace(VecRef vector, float scale);
  void MatrixUpdate(MatRef weights, MatView gradients, float learningRate);
  void VectorUpdate(VecRef weights, VecView gradients, float learningRate);

  // ---- capabilities with no IAccelerationManager slot: code the reference
  // runs inline on the host in TransformerTrainer and NeuralNetwork, which a
  // HIP-aware caller reaches through an optional interface (as decode).
  // TransformerTrainer.SegmentedAttentionForwardWithCache's attention
  // (TransformerTrainer.cs:747-796): segmentCount independent sequences of
  // segmentLength rows in q, k, v [segmentCount * segmentLength, D], scale
  // 1/sqrt(d_h), keys j <= i when causal.
  Matrix SegmentedAttentionForward(MatView q, MatView k, MatView v, int numHeads, int segmentLength,
                                   int segmentCount, bool causal);
  // SegmentedMultiHeadAttentionBackward (TransformerTrainer.cs:989-1120).
  std::tuple<Matrix, Matrix, Matrix> SegmentedMultiHeadAttentionBackward(MatView Q, MatView K, MatView V,
                                                                         MatView dConcatenated, int numHeads,
                                                                         float scale, int segmentLength,
                                                                         int segmentCount, bool causal);
  // ApplySegmentedRotaryInPlace (TransformerTrainer.cs:811-848): RoPE of q and
  // k at position row % segmentLength.
  void ApplySegmentedRotaryInPlace(MatRef q, MatRef k, int numHeads, int segmentLength, bool inverse);
  // NeuralNetwork.ComputeInputGradientBatch with gradient storage
  // (NeuralNetwork.cs:773-882, AccumulateGradientsBatch :946-985): the
  // forward recomputed with its pre-activations, the deltas through every
  // layer (act' of FillActivationAndDerivative), wgrads[i] += delta^T x and
  // bgrads[i] += column sums of delta; returns the input gradient.  The
  // network's output layer must have activation None (the transformer FFN's
  // [None, act, None], TransformerBlock.cs:101-123).
  Matrix FFNInputGradientBatch(MatView input, MatView dOutput, const FeedForwardNetwork &ffn,
                               const std::vector<MatRef> &weightGradients,
                               const std::vector<VecRef> &biasGradients);

  // Optional decode capability (no IAccelerationManager counterpart: the
  // reference runs this inline in LanguageModel.DecoderSelfAttentionStep,
  // LanguageModel.cs:353-427).  q, k, v [1, D] are the step's projections
  // before RoPE.  On the device: RoPE of q and k at absolutePosition (the
  // single-row form of LanguageModel.cs:432-480, base 10000), append of k and
  // v as row absolutePosition of the layer's cache, attention of q over the
  // absolutePosition + 1 cached keys with scale 1/sqrt(d_h).  q and k are
  // rotated in place and the host caches keys/values [maxSeq, D] receive the
  // appended rows, as the reference's cache does.  The device mirror of a
  // cache is keyed by its keys array; when it does not hold exactly the rows
  // below absolutePosition it is refreshed from the host arrays.
  Matrix DecodeSelfAttention(MatRef q, MatRef k, MatView v, MatRef keys, MatRef values,
                             int absolutePosition, int numHeads);

  void Dispose();
  bool disposed() const { return disposed_; }
  cdml_stream stream();  // the manager's own stream (created on first use)

  // Resident activations: every activation array a method reads or returns
  // keeps a device copy keyed by the host array's address, with the pinned
  // staging buffer of its last transfer as the shadow of its contents (the
  // resident cache of AccelerationManagers/GPU/DeviceResidentCache.cs:44-120,
  // extended from weights to activations).  A later call that receives the
  // same array compares it with the shadow and uploads it only when the
  // host side changed.  The least recently used entries are dropped beyond
  // `bytes` of device memory (and as much pinned memory); 0 turns the cache
  // off, so every activation crosses PCIe on every call.
  void SetActivationCacheLimit(size_t bytes);
  size_t activation_cache_limit() const { return act_limit_; }
  // The cache memory of all managers of the process together is bounded too
  // (4 GiB by default): a manager over it evicts its own entries first, and
  // an array that finds no room, or whose device or pinned allocation fails
  // after eviction, is moved through the uncached scratch path instead of
  // failing the call.
  static void SetProcessActivationCacheBudget(size_t bytes);
  static size_t ProcessActivationCacheBudget();
  static size_t ProcessActivationCacheBytes();
  // Test hook: the next `count` cache allocations fail as an out-of-memory
  // cdml_malloc would.
  static void InjectActivationAllocFailures(int count);
  int activation_cache_entries();
  // Host<->device bytes this manager has moved (uploads, downloads) and how
  // many activation uploads the shadow compare saved.
  struct TransferStats {
    uint64_t h2d_bytes = 0, d2h_bytes = 0, h2d_skipped_bytes = 0;
    uint64_t backward_from_saved = 0;  // attention backwards that reused a forward's statistics
    uint64_t act_alloc_failures = 0;   // cache allocations that failed (the array went uncached or evicted more)
  };
  TransferStats transfer_stats();

 private:
  struct Resident {
    int rows = 0, cols = 0;
    void *dev = nullptr;
    std::vector<float> shadow;
  };
  struct DeviceBuf {
    void *p = nullptr;
    size_t bytes = 0;
  };
  struct DecodeMirror {
    void *k = nullptr, *v = nullptr;
    int rows = 0, cols = 0, uploaded = 0;
  };

  struct ActEntry {
    int rows = 0, cols = 0;
    void *dev = nullptr, *pin = nullptr;
    size_t cap = 0;
    uint64_t last = 0, busy = 0;
    uint64_t ver = 0;  // changes whenever the device contents may have changed
  };
  // Row statistics of an attention forward (cdml_sdpa_fwd_lse) kept for a
  // later MultiHeadAttentionBackward on the same arrays: valid while the q,
  // k, v and output entries still hold the versions they had.
  struct LseRecord {
    const float *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
    void *qd = nullptr, *kd = nullptr, *vd = nullptr, *od = nullptr;
    uint64_t qv = 0, kv = 0, vv = 0, ov = 0, last = 0;
    int batch = 0, lq = 0, lk = 0, dim = 0, heads = 0;
    float scale = 0.f;
    bool causal = false;
    void *lse = nullptr;
    size_t lse_bytes = 0;
  };
  float *lse_slot(size_t bytes);
  void lse_record(const LseRecord &r);
  const LseRecord *lse_find(const float *q, const float *k, const float *v, int batch, int lq, int lk, int dim,
                            int heads, float scale, bool causal);
  float *inplace_begin(float *host, int rows, int cols, int slot);
  void inplace_end(float *host, int rows, int cols, const float *dev);
  void inplace_fail(float *host);
  struct Xfer {  // one host<->device transfer staged through pinned memory
    void *host;
    void *dev;
    size_t bytes;
    void *pin;
  };
  // Deferred shadow compares: while defer_ is set, act_in and resident hand
  // out the device copy of a known array at once and record the compare;
  // settle() runs the compares after the kernel was launched (so they
  // overlap its execution), uploads what changed and returns false when
  // anything did, in which case the caller launches again.  Only methods
  // whose kernels write nothing but their results use it.
  struct Pending {
    const void *host;
    void *shadow;  // pinned shadow of an activation, or a weight's host shadow
    void *dev;
    size_t bytes;
    bool weight;
  };
  bool settle();
  void begin_call();
  void *stage_region(size_t bytes);
  void stage_upload(void *dev, const void *host, size_t bytes, void *pin);
  void download_all(const std::vector<Xfer> &xs);
  // on `st` (the manager's stream when null), with chunk events from index ev0
  void download_enqueue(const std::vector<Xfer> &xs, cdml_stream st = nullptr, size_t ev0 = 0);
  void download_finish(const std::vector<Xfer> &xs, size_t ev0 = 0);
  cdml_stream copy_stream();
  const float *act_in(MatView m, int slot);
  float *act_inplace(MatRef m, int slot);
  float *act_out(float *host, int rows, int cols, int slot);
  float *act_out(Matrix &out, int slot) { return act_out(out.ptr(), out.rows, out.cols, slot); }
  struct Out {  // a result: host array and the device buffer it is downloaded from
    float *host;
    size_t floats;
    const float *dev;
  };
  static Out out_of(Matrix &m, const float *dev) { return Out{m.ptr(), m.data.size(), dev}; }
  void act_done(std::initializer_list<Out> outs);
  std::vector<Xfer> act_transfers(std::initializer_list<Out> outs);
  void launch_settle_download(const std::function<void()> &launch, std::initializer_list<Out> outs);
  void launch_split_download(const std::function<void(int, int)> &launch_rows, int rows, int h,
                             std::initializer_list<Out> outs, const std::function<void()> &before_finish);
  ActEntry act_acquire(size_t bytes);  // dev == nullptr: no cache memory, take the scratch path
  void act_release(const ActEntry &e);
  void act_destroy(const ActEntry &e);
  bool inplace_overlapped(MatRef m, const std::function<void(float *)> &launch);
  void *spare_pin(size_t cap);
  void spare_put(void *p, size_t cap);
  void act_drop(const float *key);
  void ensure_ready();
  void *scratch(int slot, size_t bytes);
  void *try_scratch(int slot, size_t bytes);
  const float *resident(const float *host, int rows, int cols);
  void upload(void *dev, const void *host, size_t bytes);
  void download(void *host, const void *dev, size_t bytes);
  void sync();
  Matrix attention(MatView q, MatView k, MatView v, int numHeads, float scale, MaskView mask,
                   bool causal, int batch = 1);
  Matrix linear(MatView x, int rowStart, int rowCount, MatView w, VecView b, int act);
  std::tuple<Matrix, Matrix, Matrix> attention_backward(MatView Q, MatView K, MatView V,
                                                        MatView dO, int numHeads, float scale,
                                                        MaskView mask, bool causal, int batch = 1);
  float elementwise_norm(const float *host, int rows, int cols);
  void elementwise_inplace(float *host, int rows, int cols, const float *src, int op, float a);
  void linear_backward(MatView x, MatView dy, int rows, MatView w, MatRef wgrad, VecRef bgrad,
                       float *dx_host, bool accumulate_dx);

  int device_;
  bool ready_ = false, disposed_ = false;
  cdml_stream stream_ = nullptr;
  cdml_stream copy_ = nullptr;     // downloads that overlap the next kernel (created on first use)
  cdml_event kev_[2] = {nullptr, nullptr};  // ends of the kernel parts those downloads wait for
  std::mutex mu_;
  std::unordered_map<const float *, Resident> resident_;
  std::vector<DeviceBuf> scratch_;
  std::unordered_map<const float *, DecodeMirror> decode_;
  // pinned staging: a grow-only buffer handed out front to back within a call
  void *stage_ = nullptr;
  size_t stage_cap_ = 0, stage_off_ = 0;
  std::vector<cdml_event> events_;
  bool dirty_ = false;  // work enqueued since the last synchronisation
  bool defer_ = false;
  std::vector<Pending> pending_;
  std::unordered_map<const float *, ActEntry> acts_;
  std::multimap<size_t, ActEntry> act_free_;
  std::vector<ActEntry> act_parked_;  // dropped while this call used them; released when it ends
  std::multimap<size_t, void *> pin_spare_;  // idle pinned buffers that in-place calls swap with shadows
  size_t act_held_ = 0, act_limit_ = size_t(1) << 30;
  uint64_t tick_ = 0, call_ = 0, ver_ = 0;
  TransferStats stats_;
  std::vector<LseRecord> lse_;  // at most kLseRecords, least recently used replaced
  void *lse_spare_ = nullptr;   // the buffer the next record will take
  size_t lse_spare_bytes_ = 0;
  std::vector<DeviceBuf> ffn_scratch_;  // FFNInputGradientBatch's per-layer buffers
};

// ---- the MultiTypeTransformer classes on the manager ----------------------
struct TransformerConfig {
  int VocabSize = 50000;
  int MaxSequenceLength = 512;
  int EmbeddingDim = 512;
  int NumHeads = 8;
  int NumLayers = 6;
  int FeedForwardDim = 2048;
  bool UseDecoderOnly = true;
  bool UsesDiscreteTokens = true;
  int InputFeatureDim = 1;
  int OutputDim = 1;
  int FFNActivationType = Relu;
  // Carried through config.json (LanguageModel.cs:710-728) and the FFN files;
  // no effect on the forward pass.  DataType is TransformerDataType
  // (Text 0, TimeSeriesRegression 1, TimeSeriesClassification 2,
  // SymbolicSequence 3; discrete tokens for 0 and 3).  AccelerationType 4 is
  // the HIP manager appended to the reference's enum.
  int DataType = 0;
  int AccelerationType = 4;
  int AccelerationDeviceId = 0;
  float L2RegulationLamda = 0.01f;
  float GradientClippingThreshold = 1.0f;
  int CostFunction = 0;
  int ActivationDistribution = 0;
  int EffectiveOutputDim() const { return UsesDiscreteTokens ? VocabSize : OutputDim; }
  void Validate() const;  // TransformerConfig.cs:62-102
};

class MultiHeadAttention {  // MultiHeadAttention.cs:6-159
 public:
  MultiHeadAttention(int embeddingDim, int numHeads, HipAccelerationManager *accel);
  Matrix Forward(MatView input, MaskView mask = {}, bool causal = false);
  Matrix WQ, WK, WV, WO;
  std::vector<float> BiasQ, BiasK, BiasV, BiasO;
  int embedding_dim() const { return dim_; }
  int num_heads() const { return heads_; }

 private:
  int dim_, heads_, head_dim_;
  HipAccelerationManager *accel_;
};

class TransformerBlock {  // TransformerBlock.cs:35-136
 public:
  TransformerBlock(int embeddingDim, int numHeads, int feedForwardDim, int ffnActivation,
                   HipAccelerationManager *accel);
  Matrix Forward(MatView x, MaskView selfMask = {}, bool causal = false);
  MultiHeadAttention Attention;
  FeedForwardNetwork FeedForward;
  std::vector<float> LN1Gamma, LN1Beta, LN2Gamma, LN2Beta;

 private:
  HipAccelerationManager *accel_;
};

// LanguageModel.cs restated: Forward (:112-233) and Generate (:482-537), the
// latter feeding the prompt token by token through per-layer host KV caches
// (:270-480) with the attention itself on the manager's decode capability.
class LanguageModel {
 public:
  LanguageModel(const TransformerConfig &cfg, HipAccelerationManager *accel);
  Matrix Forward(const std::vector<int> &tokenIds);
  Matrix Forward(MatView inputSequence);  // continuous inputs (InputProjection)
  // ForwardTokenSlice / ForwardContinuousSlice (LanguageModel.cs:135-157):
  // the forward pass of rows [start, start + count) of a sequence, which the
  // trainer's Validate / ValidateContinuous call.
  Matrix ForwardTokenSlice(const std::vector<int> &tokenIds, int tokenStart, int tokenCount);
  Matrix ForwardContinuousSlice(MatView inputSequence, int rowStart, int rowCount);
  // Greedy: argmax with the lowest index on ties.  Otherwise logits / T are
  // sampled with the SplitMix64 stream seeded by `seed` (the reference uses
  // System.Random, which this does not reproduce).
  std::vector<int> Generate(const std::vector<int> &prompt, int maxNewTokens,
                            float temperature = 1.0f, bool greedy = true, uint64_t seed = 0);
  std::vector<float> PredictNext(MatView inputSequence);
  const TransformerConfig &config() const { return cfg_; }
  HipAccelerationManager *AccelerationManager() const { return accel_; }  // LanguageModel.cs:17
  // LanguageModel.Save / Load (LanguageModel.cs:706-839): config.json,
  // weights.bin and ffn/ffn_layer_<i>.json in the reference's formats.
  void Save(const std::string &directory) const;
  static LanguageModel Load(const std::string &directory, HipAccelerationManager *accel);

  Matrix TokenEmbedding, InputProjection, OutputProjection;
  std::vector<float> InputProjectionBias, OutputBias;
  std::vector<TransformerBlock> Blocks;

 private:
  struct LayerCache {
    Matrix Keys, Values;
    int Length = 0;
  };
  Matrix ForwardHidden(Matrix x);
  Matrix ProjectToOutput(const Matrix &hidden);
  std::vector<float> ProjectLastTokenOnly(const Matrix &hidden);
  Matrix DecoderTokenStep(int tokenId, int absolutePosition, std::vector<LayerCache> &caches);
  Matrix DecoderSelfAttentionStep(MultiHeadAttention &attn, const Matrix &input,
                                  int absolutePosition, LayerCache &cache);
  int NextToken(const std::vector<float> &logits, float temperature, bool greedy,
                uint64_t &rng_state) const;
  void ValidateTokenSequence(const std::vector<int> &ids) const;

  TransformerConfig cfg_;
  HipAccelerationManager *accel_;
};

// ---- device-resident engine ----------------------------------------------
class DeviceLanguageModel {
 public:
  // Uploads every weight of `model` once; the model's arrays are not read
  // again.  batch_capacity / the config's MaxSequenceLength size the HBM
  // activations and the KV caches.
  DeviceLanguageModel(const LanguageModel &model, int batch_capacity, int device = 0);
  ~DeviceLanguageModel();
  DeviceLanguageModel(const DeviceLanguageModel &) = delete;
  DeviceLanguageModel &operator=(const DeviceLanguageModel &) = delete;

  // Discrete tokens: ids [batch, seqLen] -> logits [batch * seqLen, outputDim].
  Matrix Forward(const std::vector<int> &ids, int batch, int seqLen);
  // Continuous inputs: x [batch * seqLen, InputFeatureDim] -> [batch * seqLen, outputDim].
  Matrix ForwardContinuous(MatView x, int batch, int seqLen);
  // Greedy generation for `batch` prompts of equal length promptLen (ids
  // [batch, promptLen]); returns [batch, promptLen + n] with n =
  // min(maxNewTokens, MaxSequenceLength - promptLen) (0 when promptLen >=
  // MaxSequenceLength), the count the reference's Generate produces.
  std::vector<int> GenerateGreedy(const std::vector<int> &prompts, int batch, int promptLen,
                                  int maxNewTokens, int *outLen);
  // Enqueue-only forms over device pointers for benchmarking.
  void forward_device(const int *dev_ids, const float *dev_x, int batch, int seqLen,
                      float *dev_out);
  // The decoder blocks alone, in place on device rows x [batch * seqLen, D].
  void layers_device(float *dev_x, int batch, int seqLen);
  cdml_stream stream() const { return stream_; }
  int output_dim() const { return cfg_.EffectiveOutputDim(); }
  int batch_capacity() const { return cap_; }
  void synchronize();
  // GenerateGreedy records its device work (prefill, every decode step,
  // the token choices) once per (batch, promptLen, n) and replays it as one
  // graph launch; off, every kernel is launched from the host.
  bool use_graphs = true;
  // Decode steps of a small model (cdml_tiny_decode's limits) run in one
  // fused launch; off, each step runs the per-kernel path.
  bool use_fused_decode = true;
  bool fused_decode_available() const { return tiny_ok_; }

 private:
  struct Layer {
    float *wq, *wk, *wv, *wo, *bq, *bk, *bv, *bo;
    float *ln1g, *ln1b, *ln2g, *ln2b;
    std::vector<float *> ffw, ffb;
    std::vector<int> ffrows, ffcols, ffact;
    float *kcache, *vcache;  // [batch_capacity, maxSeq, D]
  };
  float *alloc(size_t floats);
  float *upload(const float *host, size_t floats);
  void hidden_pass(float *x, int batch, int seqLen, bool fill_cache);
  void decode_step(const int *dev_tok, int batch, int pos, float *x);
  void generate_device(int batch, int promptLen, int n);

  TransformerConfig cfg_;
  int cap_, device_;
  cdml_stream stream_ = nullptr;
  std::vector<void *> allocs_;
  std::vector<Layer> layers_;
  float *emb_ = nullptr, *inproj_ = nullptr, *inbias_ = nullptr, *outproj_ = nullptr,
        *outbias_ = nullptr;
  // activations [cap * maxSeq, width]
  float *x_, *q_, *k_, *v_, *att_, *proj_, *h_, *ff_, *ff2_, *logits_;
  int *ids_, *pos_, *kvlen_, *gen_;
  float *rope_cs_;  // cdml_rope_table of MaxSequenceLength positions
  void *ws_ = nullptr;
  size_t ws_bytes_ = 0;
  int ff_max_ = 0;
  std::map<std::tuple<int, int, int, bool>, cdml_graph> graphs_;  // (batch, promptLen, n, fused decode)
  cdml_tiny_model tiny_{};  // descriptors for cdml_tiny_decode (layers in device memory)
  bool tiny_ok_ = false;
};

// ---- the reference's trainer on the manager -------------------------------
// TrainingConfig (Transformers/Configuration/SharedConfigs.cs:24-60) is below.
struct TrainingConfig;

// Transformers/MultiTypeTransformer/TransformerTrainer.cs restated on
// HipAccelerationManager, call for call, for token models (Train,
// TrainBatchDiscrete, Validate) and continuous-input models (TrainContinuous,
// TrainBatchContinuous, ValidateContinuous): every
// `_accel.X(...)` of the reference is the manager's X with host arrays in and
// out (resident on the device between calls), the trainer's own host loops
// (the sparse row tracker of the token-embedding gradient, ScaleMatrixLocal,
// MatrixAllFinite, TransformerGradients.Zero) stay host loops as in the
// reference, and the three pieces the reference runs inline on the host
// (segmented attention forward and backward, segmented RoPE) and the FFN's
// NeuralNetwork.ComputeInputGradientBatch go to the manager's capability
// methods.  The model's host arrays are updated in place, as the reference's
// are.
class TransformerTrainer {
 public:
  TransformerTrainer(LanguageModel &model, const TrainingConfig &config);
  ~TransformerTrainer();
  // TrainBatchDiscrete(batch, 0, batch.Length, learningRate) (:217-327).
  float TrainBatch(const std::vector<std::vector<int>> &batch, float learningRate);
  // Train (:43-128) with the SplitMix64 shuffle seeded by `seed`; with
  // validation sequences, Validate runs after every ValidationInterval-th
  // batch of an epoch and its losses are kept (validation_losses()).
  // Returns the last epoch's mean batch loss.
  float Train(const std::vector<std::vector<int>> &sequences, uint64_t seed = 0,
              const std::vector<std::vector<int>> *validationSequences = nullptr);
  // TrainBatchContinuous(batchIndices, 0, count, ...) (:329-512) over every
  // window of `inputs` in order: window i is inputs[i] [T_i, InputFeatureDim]
  // (an empty matrix stands for a null entry); regression models
  // (TimeSeriesRegression) read regressionTargets[i] [>= T_i, OutputDim],
  // classification models classTargets[i] (>= T_i ids); row t's target is
  // step t + 1.
  float TrainBatchContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> *regressionTargets,
                             const std::vector<std::vector<int>> *classTargets, float learningRate);
  // TrainContinuous (:130-207): epochs of SplitMix64-shuffled batches of the
  // windows with at least 2 steps.  The reference takes validation arrays
  // here and never reads them, so this form has none.
  float TrainContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> *regressionTargets,
                        const std::vector<std::vector<int>> *classTargets, uint64_t seed = 0);
  // Validate (:1142-1182) / ValidateContinuous (:1183-1267): the mean loss
  // per predicted row over the usable sequences, forward passes through
  // LanguageModel.ForwardTokenSlice / ForwardContinuousSlice.
  float Validate(const std::vector<std::vector<int>> &validationSequences);
  float ValidateContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> *regressionTargets,
                           const std::vector<std::vector<int>> *classTargets);
  float last_norm() const { return last_norm_; }
  const std::vector<float> &validation_losses() const { return val_losses_; }

  struct AttentionGradients {  // AttentionGradients.cs:9-60
    Matrix WQ_Grad, WK_Grad, WV_Grad, WO_Grad;
    std::vector<float> BiasQ_Grad, BiasK_Grad, BiasV_Grad, BiasO_Grad;
  };
  struct LayerNormGradients {  // LayerNormGradients.cs:10-40
    std::vector<float> GammaGrad, BetaGrad;
  };
  // TransformerGradients.cs:11-160 with its SparseRowGradientTracker
  // (Transformers/Utils/SparseRowGradientTracker.cs): touched embedding rows
  // in first-use order (a HashSet without removals enumerates that way).
  struct Gradients {
    Matrix TokenEmbeddingGrad, OutputProjectionGrad;
    std::vector<float> OutputBiasGrad;
    Matrix InputProjectionGrad;  // continuous models: [EmbeddingDim, InputFeatureDim]
    std::vector<float> InputProjectionBiasGrad;
    std::vector<AttentionGradients> AttentionGrads;
    std::vector<LayerNormGradients> LN1Grads, LN2Grads;
    std::vector<int> rows;
    std::vector<uint8_t> marked;
  };
  const Gradients &gradients() const { return grads_; }
  const std::vector<std::vector<Matrix>> &ffn_weight_gradients() const { return ffnWeightGrads_; }
  const std::vector<std::vector<std::vector<float>>> &ffn_bias_gradients() const { return ffnBiasGrads_; }

 private:
  using MatPtr = std::shared_ptr<Matrix>;
  struct AttentionCache {  // AttentionCache.cs
    MatPtr Input, Q, K, V, AttentionOutput;
    bool IsSegmented = false, Causal = false;
    int SegmentLength = 0, SegmentCount = 1;
  };
  struct LayerNormCache {
    MatPtr Input, Normalized;
    std::vector<float> Mean, Variance;
  };
  struct ForwardCache {  // ForwardCache.cs
    std::vector<AttentionCache> AttentionCaches;
    std::vector<LayerNormCache> LN1Caches, LN2Caches;
    std::vector<MatPtr> LayerInputs, FFNInputs, FFNOutputs;
    MatPtr EmbeddedInput, FinalHiddenStates;
    std::vector<int> TokenIds;
    int TokenStart = 0, TokenCount = 0;
    // the continuous input the embedding was projected from: the caller's
    // window, or the bucket's flattened copy (held by ContinuousOwned)
    MatView ContinuousInput;
    MatPtr ContinuousOwned;
    int ContinuousInputRowStart = 0, ContinuousInputRowCount = 0;
  };
  Matrix ForwardWithCacheDiscrete(const std::vector<int> &tokenIds, int tokenStart, int tokenCount,
                                  ForwardCache &cache);
  Matrix ForwardWithCacheDiscreteBatch(const std::vector<std::vector<int>> &sequences,
                                       const std::vector<int> &offsets, int inputLen, ForwardCache &cache);
  float TrainBatchContinuousRange(const std::vector<int> &batchIndices, int start, int count,
                                  const std::vector<Matrix> &allInputs, const std::vector<Matrix> *allRegTargets,
                                  const std::vector<std::vector<int>> *allClassTargets, float learningRate);
  bool RegressionTargetIsValid(const std::vector<Matrix> *targets, int idx, int seqLen) const;
  bool ClassTargetIsValid(const std::vector<std::vector<int>> *targets, int idx, int seqLen) const;
  Matrix ForwardWithCacheContinuous(MatView inputSequence, int rowStart, int rowCount, ForwardCache &cache);
  Matrix ForwardWithCacheContinuousBatch(const std::vector<int> &sourceIndices, const std::vector<Matrix> &allInputs,
                                         int inputLen, ForwardCache &cache);
  Matrix ForwardFromEmbeddingWithCache(MatPtr embedded, int seqLen, ForwardCache &cache, int segmentLength = 0,
                                       int segmentCount = 1);
  MatPtr AttentionForwardWithCache(MultiHeadAttention &attention, const MatPtr &input, bool causal,
                                   AttentionCache &cache);
  MatPtr SegmentedAttentionForwardWithCache(MultiHeadAttention &attention, const MatPtr &input, int segmentLength,
                                            int segmentCount, bool causal, AttentionCache &cache);
  void BackpropFromOutput(Matrix &dOutput, ForwardCache &cache);
  Matrix BackpropBlock(int layer, Matrix &dOut, ForwardCache &cache);
  Matrix BackpropAttention(int layer, Matrix &dOut, AttentionCache &cache);
  void ZeroAllGradients();
  void ScaleGradients(float scale);
  float ComputeGradientNorm();
  void ClipGradients(float threshold, float totalNorm);
  void UpdateParameters(float learningRate);

  LanguageModel &model_;
  TransformerConfig cfg_;
  std::unique_ptr<TrainingConfig> tc_;
  HipAccelerationManager *accel_;
  Gradients grads_;
  std::vector<std::vector<Matrix>> ffnWeightGrads_;
  std::vector<std::vector<std::vector<float>>> ffnBiasGrads_;
  float last_norm_ = 0.f;
  std::vector<float> val_losses_;
};

// ---- device-resident training --------------------------------------------
// TrainingConfig (Transformers/Configuration/SharedConfigs.cs:24-60), the
// fields the discrete-token trainer reads.
struct TrainingConfig {
  float LearningRate = 0.0001f;
  int BatchSize = 32;
  int Epochs = 10;
  bool UseGradientClipping = true;
  float GradientClipThreshold = 1.0f;
  bool UseLearningRateDecay = false;
  float LearningRateDecay = 0.95f;
  int ValidationInterval = 100;
  bool Verbose = false;
};

// TransformerTrainer for decoder-only token models on the device
// (Transformers/MultiTypeTransformer/TransformerTrainer.cs).  Every weight and
// gradient of the model lives in HBM in two contiguous buffers; a batch step
// (TrainBatchDiscrete, :217-327) runs the forward pass with its cache, the
// cross-entropy gradient, the backward pass through every block, the
// token-embedding gradient, the global-norm clipping and the SGD update
// without leaving the device (one loss read-back per length bucket).
class DeviceTrainer {
 public:
  // batch_capacity x seq_capacity input tokens (seq_capacity <=
  // MaxSequenceLength) size the activation cache of one bucket.
  DeviceTrainer(const LanguageModel &model, const TrainingConfig &config, int batch_capacity,
                int seq_capacity, int device = 0);
  ~DeviceTrainer();
  DeviceTrainer(const DeviceTrainer &) = delete;
  DeviceTrainer &operator=(const DeviceTrainer &) = delete;

  // TrainBatchDiscrete: sequences shorter than 2 tokens or with ids outside
  // the vocabulary are skipped, the rest bucketed by length; returns the
  // average loss (0 when nothing was valid).
  float TrainBatch(const std::vector<std::vector<int>> &batch, float learningRate);
  // Train (:43-128): epochs over shuffled batches (SplitMix64 seeded by
  // `seed`; the reference's System.Random is not reproduced) with the
  // configured learning-rate decay; returns the last epoch's average loss.
  float Train(const std::vector<std::vector<int>> &sequences, uint64_t seed = 0);
  // Continuous inputs (TrainBatchContinuous, :337-485): windows [T_i,
  // InputFeatureDim]; with DataType TimeSeriesRegression (1) the targets are
  // regTargets[i] [>= T_i, OutputDim] (MSE), with TimeSeriesClassification
  // (2) class ids classTargets[i] (>= T_i); row t predicts step t + 1.
  float TrainBatchContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> &regTargets,
                             const std::vector<std::vector<int>> &classTargets, float learningRate);
  // TrainContinuous (:130-207): epochs of shuffled batches.
  float TrainContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> &regTargets,
                        const std::vector<std::vector<int>> &classTargets, uint64_t seed = 0);
  // Writes the device weights into the model's host arrays.
  void CopyWeightsTo(LanguageModel &model);
  // Current weights / the last step's gradients (after its 1/validCount and
  // clipping scales), flattened in the device layout; `offsets()` gives each
  // tensor's (offset, count) in the order of `names()`.
  std::vector<float> weights_flat();
  std::vector<float> gradients_flat();
  const std::vector<std::string> &names() const { return names_; }
  const std::vector<std::pair<size_t, size_t>> &offsets() const { return offs_; }
  float last_norm() const { return last_norm_; }
  cdml_stream stream() const { return stream_; }
  // The benchmark's form of a step: load_batch uploads one bucket of `batch`
  // sequences of seqLenPlus1 tokens; step_loaded enqueues a whole step on it
  // (zero, forward, loss, backward, norm, update) with no read-back.
  void load_batch(const int *host_tokens, int batch, int seqLenPlus1);
  void step_loaded(float learningRate);
  // load_batch for a regression model: inputs [batch, seqLenPlus1,
  // InputFeatureDim] and targets [batch, seqLenPlus1, OutputDim].
  void load_batch_continuous(const float *host_inputs, const float *host_targets, int batch, int seqLenPlus1);
  void synchronize();

 private:
  struct Layer {
    float *wq, *wk, *wv, *wo, *bq, *bk, *bv, *bo, *ln1g, *ln1b, *ln2g, *ln2b;
    float *gwq, *gwk, *gwv, *gwo, *gbq, *gbk, *gbv, *gbo, *gln1g, *gln1b, *gln2g, *gln2b;
    std::vector<float *> ffw, ffb, gffw, gffb;
    std::vector<int> ffrows, ffcols, ffact;
    // forward cache of the current bucket
    float *x, *q, *k, *v, *att, *r1, *n1, *m1, *v1, *r2, *m2, *v2;
    float *lse;  // attention row statistics of the forward (NULL: the backward recomputes them)
    std::vector<float *> z, h;  // pre-activation / activation of each FFN hidden layer
  };
  float *alloc(size_t floats);
  void zero_grads();
  void bucket_forward(int batch, int seqLen, float grad_scale, float *loss_dev);
  void bucket_backward(int batch, int seqLen);
  void upload_bucket(const std::vector<const std::vector<int> *> &seqs, int seqLen);
  void upload_bucket_continuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> &regTargets,
                                const std::vector<std::vector<int>> &classTargets, const std::vector<int> &idx,
                                int seqLen);
  void update(int validCount, float learningRate);

  TransformerConfig cfg_;
  TrainingConfig tc_;
  int cap_b_, cap_s_, device_;
  cdml_stream stream_ = nullptr;
  std::vector<void *> allocs_;
  float *params_ = nullptr, *grads_ = nullptr;
  size_t nparams_ = 0;
  std::vector<std::string> names_;
  std::vector<std::pair<size_t, size_t>> offs_;
  void *param_table_ = nullptr;
  int param_count_ = 0;
  // emb_ / gemb_: the token embedding, or the input projection of a
  // continuous model (with inbias_ / ginbias_)
  float *emb_ = nullptr, *outproj_ = nullptr, *outbias_ = nullptr, *gemb_ = nullptr, *goutproj_ = nullptr,
        *goutbias_ = nullptr, *inbias_ = nullptr, *ginbias_ = nullptr, *inputs_ = nullptr, *regt_ = nullptr;
  std::vector<Layer> layers_;
  float *xfinal_, *logits_, *dx_, *dxa_, *dr1_, *dr2_, *dn1_, *dcat_, *dq_, *dk_, *dv_, *tmp_;
  std::vector<float *> dh_;  // FFN hidden gradients
  float *rope_cs_, *result_, *losses_;
  int *ids_, *targets_, *order_, *gstart_, *gtoken_;
  int ngroups_ = 0, loaded_b_ = 0, loaded_s_ = 0;
  void *ws_ = nullptr;
  size_t ws_bytes_ = 0;
  float last_norm_ = 0.f;
  // Every public method holds it: the trainer's device buffers and host
  // state are shared by all its calls (Train calls TrainBatch, hence
  // recursive).
  std::recursive_mutex mu_;
};

}  // namespace cdml_host
