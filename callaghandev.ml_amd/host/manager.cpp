// HipAccelerationManager: the hot-path IAccelerationManager methods on the
// gfx950 kernels of libcdml_hip.so.  Each method validates its arguments in
// the order the reference's CPU manager does (citations per method), stages
// activations through the manager's device buffers, reuses resident copies of
// weight arrays, runs the kernel(s) on the manager's stream and returns host
// arrays.  Nothing here computes on the CPU: a missing device or library is
// an InvalidOperationException.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "cdml_host.h"

namespace cdml_host {

namespace {

void check(int rc, const char *what) {
  if (rc != CDML_OK)
    throw InvalidOperationException(std::string(what) + ": " + cdml_last_error());
}

// Scratch slots of the manager's device buffer pool.
enum Slot {
  S_X = 0, S_Q, S_K, S_V, S_O, S_MASK, S_IDS, S_KVLEN, S_WS, S_BIAS,
  S_DQ, S_DK, S_DV, S_GW0, S_GW1, S_GW2, S_GB0, S_GB1, S_GB2, S_COUNT
};

}  // namespace

HipAccelerationManager::HipAccelerationManager(int device) : device_(device) {
  if (device < 0) throw ArgumentOutOfRangeException("device");
}

HipAccelerationManager::~HipAccelerationManager() {
  try {
    Dispose();
  } catch (...) {
  }
}

void HipAccelerationManager::Dispose() {
  std::lock_guard<std::mutex> lock(mu_);
  if (disposed_) return;
  disposed_ = true;
  if (!ready_) return;
  cdml_stream_synchronize(stream_);
  for (auto &kv : resident_) cdml_free(kv.second.dev);
  resident_.clear();
  for (auto &b : scratch_) cdml_free(b.p);
  scratch_.clear();
  for (auto &kv : decode_) {
    cdml_free(kv.second.k);
    cdml_free(kv.second.v);
  }
  decode_.clear();
  cdml_stream_destroy(stream_);
  stream_ = nullptr;
}

void HipAccelerationManager::ensure_ready() {
  if (disposed_) throw InvalidOperationException("HipAccelerationManager has been disposed.");
  if (ready_) return;
  check(cdml_init(device_), "cdml_init");
  check(cdml_stream_create(&stream_), "cdml_stream_create");
  scratch_.assign(S_COUNT, DeviceBuf{});
  ready_ = true;
}

cdml_stream HipAccelerationManager::stream() {
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  return stream_;
}

void *HipAccelerationManager::scratch(int slot, size_t bytes) {
  DeviceBuf &b = scratch_[slot];
  if (bytes == 0) bytes = 4;
  if (b.bytes < bytes) {
    check(cdml_stream_synchronize(stream_), "cdml_stream_synchronize");
    check(cdml_free(b.p), "cdml_free");
    b.p = nullptr;
    b.bytes = 0;
    size_t grow = bytes + bytes / 4;  // some headroom for the next, larger call
    check(cdml_malloc(&b.p, grow), "cdml_malloc");
    b.bytes = grow;
  }
  return b.p;
}

// Like scratch(), but a failed allocation returns NULL (the slot is left
// empty) instead of throwing.
void *HipAccelerationManager::try_scratch(int slot, size_t bytes) {
  DeviceBuf &b = scratch_[slot];
  if (bytes == 0) bytes = 4;
  if (b.bytes >= bytes) return b.p;
  check(cdml_stream_synchronize(stream_), "cdml_stream_synchronize");
  check(cdml_free(b.p), "cdml_free");
  b.p = nullptr;
  b.bytes = 0;
  void *p = nullptr;
  if (cdml_malloc(&p, bytes) != CDML_OK) return nullptr;
  b.p = p;
  b.bytes = bytes;
  return p;
}

size_t SdpaBackwardWorkspaceChoice(size_t base_bytes, size_t stored_ds_bytes, size_t extra_cap) {
  if (stored_ds_bytes <= base_bytes) return base_bytes;
  return stored_ds_bytes - base_bytes <= extra_cap ? stored_ds_bytes : base_bytes;
}

void HipAccelerationManager::upload(void *dev, const void *host, size_t bytes) {
  check(cdml_memcpy_h2d_async(dev, host, bytes, stream_), "cdml_memcpy_h2d_async");
}

void HipAccelerationManager::download(void *host, const void *dev, size_t bytes) {
  check(cdml_memcpy_d2h_async(host, dev, bytes, stream_), "cdml_memcpy_d2h_async");
}

void HipAccelerationManager::sync() { check(cdml_stream_synchronize(stream_), "cdml_stream_synchronize"); }

// Identity-keyed resident copy with a shadow compare
// (AccelerationManagers/GPU/DeviceResidentCache.cs:44-120): the first call
// with an array uploads it; later calls upload again only when the shape or
// the contents changed.
const float *HipAccelerationManager::resident(const float *host, int rows, int cols) {
  const size_t n = (size_t)rows * cols;
  auto it = resident_.find(host);
  if (it == resident_.end() || it->second.rows != rows || it->second.cols != cols) {
    if (it != resident_.end()) {
      sync();
      cdml_free(it->second.dev);
      resident_.erase(it);
    }
    Resident r;
    r.rows = rows;
    r.cols = cols;
    check(cdml_malloc(&r.dev, n * sizeof(float) + 4), "cdml_malloc");
    r.shadow.assign(host, host + n);
    upload(r.dev, r.shadow.data(), n * sizeof(float));
    auto res = resident_.emplace(host, std::move(r));
    return static_cast<const float *>(res.first->second.dev);
  }
  Resident &r = it->second;
  if (n && std::memcmp(r.shadow.data(), host, n * sizeof(float)) != 0) {
    sync();  // an earlier enqueued copy may still read the shadow
    std::memcpy(r.shadow.data(), host, n * sizeof(float));
    upload(r.dev, r.shadow.data(), n * sizeof(float));
  }
  return static_cast<const float *>(r.dev);
}

// ---- ProjectQKV: AccelerationCPU.cs:2005-2069 -----------------------------
std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::ProjectQKV(MatView input, MatView WQ,
                                                                      VecView biasQ, MatView WK,
                                                                      VecView biasK, MatView WV,
                                                                      VecView biasV) {
  if (input.null()) throw ArgumentNullException("input");
  if (WQ.null()) throw ArgumentNullException("WQ");
  if (WK.null()) throw ArgumentNullException("WK");
  if (WV.null()) throw ArgumentNullException("WV");
  if (biasQ.null()) throw ArgumentNullException("biasQ");
  if (biasK.null()) throw ArgumentNullException("biasK");
  if (biasV.null()) throw ArgumentNullException("biasV");
  const int rows = input.rows, inputDim = input.cols;
  const int qDim = WQ.rows, kDim = WK.rows, vDim = WV.rows;
  if (WQ.cols != inputDim) throw ArgumentException("WQ input dimension does not match input width.", "WQ");
  if (WK.cols != inputDim) throw ArgumentException("WK input dimension does not match input width.", "WK");
  if (WV.cols != inputDim) throw ArgumentException("WV input dimension does not match input width.", "WV");
  if (biasQ.length != qDim) throw ArgumentException("biasQ length does not match WQ output dimension.", "biasQ");
  if (biasK.length != kDim) throw ArgumentException("biasK length does not match WK output dimension.", "biasK");
  if (biasV.length != vDim) throw ArgumentException("biasV length does not match WV output dimension.", "biasV");
  if (qDim != kDim || qDim != vDim) throw ArgumentException("Q, K and V output dimensions must match.");

  Matrix Q(rows, qDim), K(rows, kDim), V(rows, vDim);
  if (rows == 0 || qDim == 0) return {Q, K, V};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *wq = resident(WQ.data, qDim, inputDim), *wk = resident(WK.data, kDim, inputDim),
              *wv = resident(WV.data, vDim, inputDim);
  const float *bq = resident(biasQ.data, 1, qDim), *bk = resident(biasK.data, 1, kDim),
              *bv = resident(biasV.data, 1, vDim);
  const size_t out_bytes = (size_t)rows * qDim * sizeof(float);
  float *dx = static_cast<float *>(scratch(S_X, (size_t)rows * inputDim * sizeof(float)));
  float *dq = static_cast<float *>(scratch(S_Q, out_bytes));
  float *dk = static_cast<float *>(scratch(S_K, out_bytes));
  float *dv = static_cast<float *>(scratch(S_V, out_bytes));
  upload(dx, input.data, (size_t)rows * inputDim * sizeof(float));
  check(cdml_project_qkv(dx, wq, bq, wk, bk, wv, bv, dq, dk, dv, rows, inputDim, qDim, stream_),
        "cdml_project_qkv");
  download(Q.ptr(), dq, out_bytes);
  download(K.ptr(), dk, out_bytes);
  download(V.ptr(), dv, out_bytes);
  sync();
  return {std::move(Q), std::move(K), std::move(V)};
}

// ---- attention core shared by SDPA and MultiHeadAttentionForward -----------
Matrix HipAccelerationManager::attention(MatView q, MatView k, MatView v, int numHeads,
                                         float scale, MaskView mask, bool causal) {
  const int lq = q.rows, lk = k.rows, dim = q.cols;
  Matrix out(lq, dim);
  if (lq == 0 || lk == 0 || dim == 0) return out;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t qb = (size_t)lq * dim * sizeof(float), kb = (size_t)lk * dim * sizeof(float);
  float *dq = static_cast<float *>(scratch(S_Q, qb));
  float *dk = static_cast<float *>(scratch(S_K, kb));
  float *dv = static_cast<float *>(scratch(S_V, kb));
  float *dout = static_cast<float *>(scratch(S_O, qb));
  upload(dq, q.data, qb);
  upload(dk, k.data, kb);
  upload(dv, v.data, kb);
  const uint8_t *dm = nullptr;
  if (!mask.null()) {
    void *m = scratch(S_MASK, (size_t)lq * lk);
    upload(m, mask.data, (size_t)lq * lk);
    dm = static_cast<const uint8_t *>(m);
  }
  check(cdml_sdpa_fwd(dq, dim, dk, dim, dv, dim, dout, dim, 1, lq, lk, dim, numHeads, scale,
                      causal ? 1 : 0, dm, stream_),
        "cdml_sdpa_fwd");
  download(out.ptr(), dout, qb);
  sync();
  return out;
}

// ---- ScaledDotProductAttention: AccelerationCPU.cs:1797-1956 ---------------
Matrix HipAccelerationManager::ScaledDotProductAttention(MatView q, MatView k, MatView v,
                                                         int numHeads, MaskView mask, bool causal) {
  if (q.null()) throw ArgumentNullException("q");
  if (k.null()) throw ArgumentNullException("k");
  if (v.null()) throw ArgumentNullException("v");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  const int queryLen = q.rows, keyLen = k.rows, valueLen = v.rows, dim = q.cols;
  if (queryLen <= 0) throw ArgumentException("Q must contain at least one row.", "q");
  if (keyLen <= 0) throw ArgumentException("K must contain at least one row.", "k");
  if (dim <= 0) throw ArgumentException("Q must contain at least one column.", "q");
  if (k.cols != dim) throw ArgumentException("K width must match Q width.", "k");
  if (v.cols != dim) throw ArgumentException("V width must match Q width.", "v");
  if (valueLen != keyLen) throw ArgumentException("V row count must match K row count.", "v");
  if (dim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by numHeads.", "numHeads");
  if (!mask.null() && (mask.rows != queryLen || mask.cols != keyLen))
    throw ArgumentException("Mask shape must be [" + std::to_string(queryLen) + "," +
                                std::to_string(keyLen) + "], got [" + std::to_string(mask.rows) +
                                "," + std::to_string(mask.cols) + "].",
                            "mask");
  if (causal && queryLen != keyLen)
    throw ArgumentException(
        "The simple causal path assumes queryLen == keyLen. Use an explicit mask for "
        "cross-attention or cached decoding.");
  const int headDim = dim / numHeads;
  const float scale = 1.0f / std::sqrt((float)headDim);  // AccelerationCPU.cs:1865
  return attention(q, k, v, numHeads, scale, mask, causal);
}

// ---- MultiHeadAttentionForward: AccelerationCPU.cs:1647-1792 ---------------
Matrix HipAccelerationManager::MultiHeadAttentionForward(MatView Q, MatView K, MatView V,
                                                         int numHeads, float scale, MaskView mask) {
  if (Q.null()) throw ArgumentNullException("Q");
  if (K.null()) throw ArgumentNullException("K");
  if (V.null()) throw ArgumentNullException("V");
  const int seqLenQ = Q.rows, seqLenK = K.rows, dim = Q.cols;
  if (K.cols != dim || V.cols != dim)
    throw ArgumentException("Q, K and V must have the same embedding dimension.");
  if (V.rows != seqLenK) throw ArgumentException("K and V must have the same sequence length.");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  if (dim % numHeads != 0) throw ArgumentException("Embedding dim must be divisible by numHeads.");
  if (!mask.null() && (mask.rows != seqLenQ || mask.cols != seqLenK))
    throw ArgumentException("Mask shape must be [seqLenQ, seqLenK].");
  if (seqLenQ == 0 || seqLenK == 0 || dim / numHeads == 0) return Matrix(seqLenQ, dim);
  return attention(Q, K, V, numHeads, scale, mask, false);
}

// ---- ProjectOutputBatch / BatchDotProductAddBias ---------------------------
Matrix HipAccelerationManager::linear(MatView x, int rowStart, int rowCount, MatView w, VecView b,
                                      int act) {
  const int in = w.cols, out = w.rows;
  Matrix y(rowCount, out);
  if (rowCount == 0 || out == 0) return y;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *dw = resident(w.data, out, in);
  const float *db = resident(b.data, 1, out);
  const size_t xb = (size_t)rowCount * in * sizeof(float), yb = (size_t)rowCount * out * sizeof(float);
  float *dx = static_cast<float *>(scratch(S_X, xb));
  float *dy = static_cast<float *>(scratch(S_O, yb));
  upload(dx, x.data + (size_t)rowStart * x.cols, xb);
  check(cdml_linear(dx, in, dw, db, dy, out, rowCount, in, out, act, stream_), "cdml_linear");
  download(y.ptr(), dy, yb);
  sync();
  return y;
}

// AccelerationCPU.cs:2694-2715.  The reference reads hidden[i, :] for i <
// seqLen and projection rows j < outputDim without checks (an out-of-range
// shape raises IndexOutOfRangeException there); the same shapes are rejected
// here with ArgumentException before any device work.
Matrix HipAccelerationManager::ProjectOutputBatch(MatView hidden, MatView outputProjection,
                                                  VecView outputBias, int seqLen, int outputDim) {
  if (hidden.null()) throw ArgumentNullException("hidden");
  if (outputProjection.null()) throw ArgumentNullException("outputProjection");
  if (outputBias.null()) throw ArgumentNullException("outputBias");
  if (seqLen < 0 || seqLen > hidden.rows) throw ArgumentException("seqLen exceeds the hidden rows.", "seqLen");
  if (outputDim < 0 || outputDim > outputProjection.rows || outputDim > outputBias.length)
    throw ArgumentException("outputDim exceeds the projection rows or bias length.", "outputDim");
  if (outputProjection.cols != hidden.cols)
    throw ArgumentException("Projection width must match the hidden width.", "outputProjection");
  MatView w(outputProjection.data, outputDim, outputProjection.cols);
  return linear(hidden, 0, seqLen, w, VecView(outputBias.data, outputDim), CDML_ACT_NONE);
}

Matrix HipAccelerationManager::BatchDotProductAddBias(MatView weights, MatView inputMatrix,
                                                      VecView bias) {
  if (inputMatrix.null()) throw ArgumentNullException("inputMatrix");
  return BatchDotProductAddBias(weights, inputMatrix, 0, inputMatrix.rows, bias);
}

// AccelerationCPU.cs:352-404
Matrix HipAccelerationManager::BatchDotProductAddBias(MatView weights, MatView inputMatrix,
                                                      int rowStart, int rowCount, VecView bias) {
  if (weights.null()) throw ArgumentNullException("weights");
  if (inputMatrix.null()) throw ArgumentNullException("inputMatrix");
  if (bias.null()) throw ArgumentNullException("bias");
  if (rowStart < 0 || rowCount < 0 || (long long)rowStart + rowCount > inputMatrix.rows)
    throw ArgumentOutOfRangeException("rowStart");
  if (inputMatrix.cols != weights.cols)
    throw ArgumentException("Expected input columns " + std::to_string(weights.cols) + ", got " +
                                std::to_string(inputMatrix.cols),
                            "inputMatrix");
  if (bias.length != weights.rows) throw ArgumentException("Bias length must match output dimension.", "bias");
  if (rowCount == 0 || weights.rows == 0 || weights.cols == 0) {
    Matrix y(rowCount, weights.rows);
    if (weights.cols == 0)  // an empty dot product leaves only the bias
      for (int i = 0; i < rowCount; ++i)
        for (int j = 0; j < weights.rows; ++j) y.at(i, j) = bias.data[j];
    return y;
  }
  return linear(inputMatrix, rowStart, rowCount, weights, bias, CDML_ACT_NONE);
}

// ---- RoPE: AccelerationCPU.cs:4855-4982 --------------------------------------
void HipAccelerationManager::ApplyRotaryPositionEmbeddingInPlace(MatRef matrix, int numHeads,
                                                                 float baseTheta, bool inverse) {
  if (!matrix.data) throw ArgumentNullException("matrix");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  if (!(baseTheta > 0.f) || std::isinf(baseTheta)) throw ArgumentOutOfRangeException("baseTheta");
  const int dim = matrix.cols;
  if (dim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by number of heads.");
  const int headDim = dim / numHeads;
  if (headDim & 1) throw ArgumentException("RoPE requires an even per-head dimension.");
  if (matrix.rows == 0 || headDim == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t bytes = (size_t)matrix.rows * dim * sizeof(float);
  float *dx = static_cast<float *>(scratch(S_X, bytes));
  upload(dx, matrix.data, bytes);
  check(cdml_rope(dx, matrix.rows, dim, 0, headDim, numHeads, baseTheta, inverse ? 1 : 0, 0, 0,
                  nullptr, stream_),
        "cdml_rope");
  download(matrix.data, dx, bytes);
  sync();
}

void HipAccelerationManager::ApplyRotaryPositionEmbeddingHeadInPlace(MatRef matrix, int startCol,
                                                                     int headDim, float baseTheta,
                                                                     bool inverse) {
  if (!matrix.data) throw ArgumentNullException("matrix");
  if (startCol < 0) throw ArgumentOutOfRangeException("startCol");
  if (headDim < 0) throw ArgumentOutOfRangeException("headDim");
  if (headDim & 1) throw ArgumentException("RoPE requires an even per-head dimension.", "headDim");
  if (!(baseTheta > 0.f) || std::isinf(baseTheta)) throw ArgumentOutOfRangeException("baseTheta");
  if ((long long)startCol + headDim > matrix.cols)
    throw ArgumentException("Head range exceeds matrix embedding dimension.");
  if (matrix.rows == 0 || headDim == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t bytes = (size_t)matrix.rows * matrix.cols * sizeof(float);
  float *dx = static_cast<float *>(scratch(S_X, bytes));
  upload(dx, matrix.data, bytes);
  check(cdml_rope(dx, matrix.rows, matrix.cols, startCol, headDim, 1, baseTheta, inverse ? 1 : 0,
                  0, 0, nullptr, stream_),
        "cdml_rope");
  download(matrix.data, dx, bytes);
  sync();
}

// ---- ResidualLayerNorm: AccelerationCPU.cs:1376-1438 ----------------------
Matrix HipAccelerationManager::ResidualLayerNorm(MatView input, MatView subLayer, VecView gamma,
                                                 VecView beta, float epsilon) {
  if (input.null()) throw ArgumentNullException("input");
  if (subLayer.null()) throw ArgumentNullException("subLayer");
  if (gamma.null()) throw ArgumentNullException("gamma");
  if (beta.null()) throw ArgumentNullException("beta");
  const int rows = input.rows, f = input.cols;
  if (subLayer.rows != rows || subLayer.cols != f)
    throw ArgumentException("Residual input dimensions must match.", "subLayer");
  if (gamma.length != f || beta.length != f)
    throw ArgumentException("Layer norm gamma/beta must match the feature dimension.");
  Matrix out(rows, f);
  if (rows == 0 || f == 0) return out;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t bytes = (size_t)rows * f * sizeof(float);
  const float *dg = resident(gamma.data, 1, f), *db = resident(beta.data, 1, f);
  float *da = static_cast<float *>(scratch(S_X, bytes));
  float *dbb = static_cast<float *>(scratch(S_Q, bytes));
  float *dy = static_cast<float *>(scratch(S_O, bytes));
  upload(da, input.data, bytes);
  upload(dbb, subLayer.data, bytes);
  check(cdml_residual_layernorm(da, dbb, dg, db, dy, rows, f, epsilon, stream_),
        "cdml_residual_layernorm");
  download(out.ptr(), dy, bytes);
  sync();
  return out;
}

// ---- EmbedTokenIds: AccelerationCPU.cs:3463-3515 --------------------------
Matrix HipAccelerationManager::EmbedTokenIds(const std::vector<int> &tokenIds, MatView embedding,
                                             int embeddingDim) {
  if (tokenIds.empty()) return Matrix(0, embeddingDim);
  return EmbedTokenIds(tokenIds, 0, (int)tokenIds.size(), embedding, embeddingDim);
}

Matrix HipAccelerationManager::EmbedTokenIds(const std::vector<int> &tokenIds, int tokenStart,
                                             int tokenCount, MatView embedding, int embeddingDim) {
  if (tokenIds.empty() || tokenCount == 0) return Matrix(0, embeddingDim);
  if (embedding.null()) throw ArgumentNullException("embedding");
  if (tokenStart < 0 || tokenCount < 0 || (long long)tokenStart + tokenCount > (long long)tokenIds.size())
    throw ArgumentOutOfRangeException("tokenStart");
  const int vocab = embedding.rows;
  if (embedding.cols != embeddingDim) throw ArgumentException("Embedding dimension mismatch.", "embedding");
  for (int i = 0; i < tokenCount; ++i) {
    const int t = tokenIds[tokenStart + i];
    if ((unsigned)t >= (unsigned)vocab)
      throw ArgumentOutOfRangeException("tokenIds", "Token out of range: " + std::to_string(t));
  }
  Matrix out(tokenCount, embeddingDim);
  if (embeddingDim == 0) return out;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const float *dt = resident(embedding.data, vocab, embeddingDim);
  int *dids = static_cast<int *>(scratch(S_IDS, (size_t)tokenCount * sizeof(int)));
  float *dout = static_cast<float *>(scratch(S_O, (size_t)tokenCount * embeddingDim * sizeof(float)));
  upload(dids, tokenIds.data() + tokenStart, (size_t)tokenCount * sizeof(int));
  check(cdml_embed_tokens(dids, tokenCount, dt, vocab, embeddingDim, dout, nullptr, stream_),
        "cdml_embed_tokens");
  download(out.ptr(), dout, (size_t)tokenCount * embeddingDim * sizeof(float));
  sync();
  return out;
}

// ---- CreateCausalMask: AccelerationCPU.cs:1566-1586 (host data only) --------
BoolMatrix HipAccelerationManager::CreateCausalMask(int seqLen) {
  if (seqLen < 0) throw ArgumentOutOfRangeException("seqLen");
  BoolMatrix m;
  m.rows = m.cols = seqLen;
  m.data.assign((size_t)seqLen * seqLen, 0);
  for (int i = 0; i < seqLen; ++i)
    for (int j = 0; j <= i; ++j) m.data[(size_t)i * seqLen + j] = 1;
  return m;
}

// ---- FFNForwardBatch: AccelerationCPU.cs:1957-2002 + NeuralNetwork.cs:629-668
Matrix HipAccelerationManager::FFNForwardBatch(MatView input, int seqLen, int outputDim,
                                               const FeedForwardNetwork &ffn) {
  if (input.null()) throw ArgumentNullException("input");
  if (seqLen < 0 || seqLen > input.rows) throw ArgumentOutOfRangeException("seqLen");
  if (ffn.weights.empty()) throw InvalidOperationException("Neural network must have at least input and output layers.");
  if (seqLen == 0) return Matrix(0, ffn.output_size());
  if (input.cols != ffn.input_size())
    throw ArgumentException("Input matrix column count (" + std::to_string(input.cols) +
                                ") must match network input size (" +
                                std::to_string(ffn.input_size()) + ").",
                            "input");
  (void)outputDim;  // the reference's batched route returns the network's own output width
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  int width = input.cols;
  size_t maxw = width;
  for (auto &w : ffn.weights) maxw = std::max(maxw, (size_t)w.rows);
  float *a = static_cast<float *>(scratch(S_X, (size_t)seqLen * maxw * sizeof(float)));
  float *b = static_cast<float *>(scratch(S_O, (size_t)seqLen * maxw * sizeof(float)));
  upload(a, input.data, (size_t)seqLen * width * sizeof(float));
  for (size_t l = 0; l < ffn.weights.size(); ++l) {
    const Matrix &w = ffn.weights[l];
    if (w.cols != width) throw ArgumentException("FFN layer widths do not chain.", "ffn");
    if ((int)ffn.biases[l].size() != w.rows) throw ArgumentException("FFN bias length mismatch.", "ffn");
    const float *dw = resident(w.ptr(), w.rows, w.cols);
    const float *db = resident(ffn.biases[l].data(), 1, w.rows);
    check(cdml_linear(a, width, dw, db, b, w.rows, seqLen, width, w.rows, ffn.activations[l], stream_),
          "cdml_linear");
    std::swap(a, b);
    width = w.rows;
  }
  Matrix out(seqLen, width);
  download(out.ptr(), a, (size_t)seqLen * width * sizeof(float));
  sync();
  return out;
}

// ---- MultiHeadAttentionBackward: AccelerationCPU.cs:1011-1280 ----------------
std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::MultiHeadAttentionBackward(
    MatView Q, MatView K, MatView V, MatView dConcatenated, int numHeads, float scale,
    bool useDecoderMask) {
  return attention_backward(Q, K, V, dConcatenated, numHeads, scale, MaskView{}, useDecoderMask);
}

std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::MultiHeadAttentionBackward(
    MatView Q, MatView K, MatView V, MatView dConcatenated, int numHeads, float scale,
    MaskView mask) {
  return attention_backward(Q, K, V, dConcatenated, numHeads, scale, mask, false);
}

// MultiHeadAttentionBackwardCore's checks (AccelerationCPU.cs:1037-1063) in
// order, then cdml_sdpa_bwd on the manager's stream.
std::tuple<Matrix, Matrix, Matrix> HipAccelerationManager::attention_backward(
    MatView Q, MatView K, MatView V, MatView dO, int numHeads, float scale, MaskView mask,
    bool causal) {
  if (Q.null()) throw ArgumentNullException("Q");
  if (K.null()) throw ArgumentNullException("K");
  if (V.null()) throw ArgumentNullException("V");
  if (dO.null()) throw ArgumentNullException("dConcatenated");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads");
  const int lq = Q.rows, lk = K.rows, dim = Q.cols;
  if (K.cols != dim || V.cols != dim)
    throw ArgumentException("Q, K and V must have the same embedding dimension.");
  if (V.rows != lk) throw ArgumentException("K and V must have the same sequence length.");
  if (dO.rows != lq || dO.cols != dim)
    throw ArgumentException("dConcatenated shape must match Q shape.", "dConcatenated");
  if (dim % numHeads != 0)
    throw ArgumentException("Embedding dim must be divisible by numHeads.", "numHeads");
  if (!mask.null() && (mask.rows != lq || mask.cols != lk))
    throw ArgumentException("Mask shape must be [" + std::to_string(lq) + "," + std::to_string(lk) +
                                "], got [" + std::to_string(mask.rows) + "," +
                                std::to_string(mask.cols) + "].",
                            "mask");
  Matrix dQ(lq, dim), dK(lk, dim), dV(lk, dim);
  if (lq == 0 || lk == 0 || dim == 0) return {std::move(dQ), std::move(dK), std::move(dV)};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t qb = (size_t)lq * dim * sizeof(float), kb = (size_t)lk * dim * sizeof(float);
  float *dq_in = static_cast<float *>(scratch(S_Q, qb));
  float *dk_in = static_cast<float *>(scratch(S_K, kb));
  float *dv_in = static_cast<float *>(scratch(S_V, kb));
  float *ddo = static_cast<float *>(scratch(S_O, qb));
  float *gq = static_cast<float *>(scratch(S_DQ, qb));
  float *gk = static_cast<float *>(scratch(S_DK, kb));
  float *gv = static_cast<float *>(scratch(S_DV, kb));
  size_t base_ws = 0, stored_ws = 0;
  check(cdml_sdpa_bwd_workspace_size(1, lq, lk, dim, numHeads, &base_ws), "cdml_sdpa_bwd_workspace_size");
  // with room for the dS blocks when the shape can use them (dQ as one
  // product), as long as the extra bytes stay under the cap and allocate
  check(cdml_sdpa_bwd_stored_ds_workspace_size(1, lq, lk, dim, numHeads, causal && mask.null() ? 1 : 0,
                                               &stored_ws),
        "cdml_sdpa_bwd_stored_ds_workspace_size");
  size_t ws = SdpaBackwardWorkspaceChoice(base_ws, stored_ws, kStoredDsExtraBytesCap);
  void *dws = ws > base_ws ? try_scratch(S_WS, ws) : nullptr;
  if (!dws) {
    ws = base_ws;
    dws = scratch(S_WS, ws);
  }
  upload(dq_in, Q.data, qb);
  upload(dk_in, K.data, kb);
  upload(dv_in, V.data, kb);
  upload(ddo, dO.data, qb);
  const uint8_t *dm = nullptr;
  if (!mask.null()) {
    void *m = scratch(S_MASK, (size_t)lq * lk);
    upload(m, mask.data, (size_t)lq * lk);
    dm = static_cast<const uint8_t *>(m);
  }
  check(cdml_sdpa_bwd(dq_in, dim, dk_in, dim, dv_in, dim, ddo, dim, gq, dim, gk, dim, gv, dim, 1,
                      lq, lk, dim, numHeads, scale, causal ? 1 : 0, dm, dws, ws, stream_),
        "cdml_sdpa_bwd");
  download(dQ.ptr(), gq, qb);
  download(dK.ptr(), gk, kb);
  download(dV.ptr(), gv, kb);
  sync();
  return {std::move(dQ), std::move(dK), std::move(dV)};
}

// ---- BackpropQKV: AccelerationCPU.cs:2071-2186 ------------------------------
Matrix HipAccelerationManager::BackpropQKV(MatView input, MatView dQ, MatView dK, MatView dV,
                                           MatView WQ, MatView WK, MatView WV, MatRef WQGrad,
                                           VecRef biasQGrad, MatRef WKGrad, VecRef biasKGrad,
                                           MatRef WVGrad, VecRef biasVGrad) {
  if (input.null()) throw ArgumentNullException("input");
  if (dQ.null()) throw ArgumentNullException("dQ");
  if (dK.null()) throw ArgumentNullException("dK");
  if (dV.null()) throw ArgumentNullException("dV");
  if (WQ.null()) throw ArgumentNullException("WQ");
  if (WK.null()) throw ArgumentNullException("WK");
  if (WV.null()) throw ArgumentNullException("WV");
  if (!WQGrad.data) throw ArgumentNullException("WQGrad");
  if (!WKGrad.data) throw ArgumentNullException("WKGrad");
  if (!WVGrad.data) throw ArgumentNullException("WVGrad");
  if (biasQGrad.null()) throw ArgumentNullException("biasQGrad");
  if (biasKGrad.null()) throw ArgumentNullException("biasKGrad");
  if (biasVGrad.null()) throw ArgumentNullException("biasVGrad");
  const int rows = input.rows, inputDim = input.cols;
  const int outputDim = WQ.rows;
  if (WK.rows != outputDim || WV.rows != outputDim)
    throw ArgumentException("Q, K and V dimensions must match.");
  if (WQ.cols != inputDim || WK.cols != inputDim || WV.cols != inputDim)
    throw ArgumentException("Q/K/V weight input dimensions must match input width.");
  if (dQ.rows != rows || dK.rows != rows || dV.rows != rows)
    throw ArgumentException("dQ, dK and dV row counts must match input row count.");
  if (dQ.cols != outputDim || dK.cols != outputDim || dV.cols != outputDim)
    throw ArgumentException("dQ, dK and dV widths must match Q/K/V output dimension.");
  if (WQGrad.rows != outputDim || WQGrad.cols != inputDim)
    throw ArgumentException("WQGrad shape mismatch.", "WQGrad");
  if (WKGrad.rows != outputDim || WKGrad.cols != inputDim)
    throw ArgumentException("WKGrad shape mismatch.", "WKGrad");
  if (WVGrad.rows != outputDim || WVGrad.cols != inputDim)
    throw ArgumentException("WVGrad shape mismatch.", "WVGrad");
  if (biasQGrad.length != outputDim || biasKGrad.length != outputDim || biasVGrad.length != outputDim)
    throw ArgumentException("Q/K/V bias gradient lengths must match output dimension.");
  Matrix dInput(rows, inputDim);
  if (rows == 0 || inputDim == 0 || outputDim == 0) return dInput;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t xb = (size_t)rows * inputDim * sizeof(float);
  const size_t db = (size_t)rows * outputDim * sizeof(float);
  const size_t wb = (size_t)outputDim * inputDim * sizeof(float), bb = (size_t)outputDim * sizeof(float);
  const float *wq = resident(WQ.data, outputDim, inputDim), *wk = resident(WK.data, outputDim, inputDim),
              *wv = resident(WV.data, outputDim, inputDim);
  float *dx_in = static_cast<float *>(scratch(S_X, xb));
  float *ddq = static_cast<float *>(scratch(S_DQ, db));
  float *ddk = static_cast<float *>(scratch(S_DK, db));
  float *ddv = static_cast<float *>(scratch(S_DV, db));
  float *ddx = static_cast<float *>(scratch(S_O, xb));
  float *gw[3] = {static_cast<float *>(scratch(S_GW0, wb)), static_cast<float *>(scratch(S_GW1, wb)),
                  static_cast<float *>(scratch(S_GW2, wb))};
  float *gb[3] = {static_cast<float *>(scratch(S_GB0, bb)), static_cast<float *>(scratch(S_GB1, bb)),
                  static_cast<float *>(scratch(S_GB2, bb))};
  MatRef hw[3] = {WQGrad, WKGrad, WVGrad};
  VecRef hb[3] = {biasQGrad, biasKGrad, biasVGrad};
  upload(dx_in, input.data, xb);
  upload(ddq, dQ.data, db);
  upload(ddk, dK.data, db);
  upload(ddv, dV.data, db);
  for (int i = 0; i < 3; ++i) {
    upload(gw[i], hw[i].data, wb);
    upload(gb[i], hb[i].data, bb);
  }
  size_t ws = 0;
  check(cdml_backprop_qkv_workspace_size(rows, inputDim, outputDim, &ws),
        "cdml_backprop_qkv_workspace_size");
  void *dws = ws ? scratch(S_WS, ws) : nullptr;
  check(cdml_backprop_qkv(dx_in, ddq, ddk, ddv, wq, wk, wv, gw[0], gb[0], gw[1], gb[1], gw[2], gb[2],
                          ddx, rows, inputDim, outputDim, dws, ws, stream_),
        "cdml_backprop_qkv");
  download(dInput.ptr(), ddx, xb);
  for (int i = 0; i < 3; ++i) {
    download(hw[i].data, gw[i], wb);
    download(hb[i].data, gb[i], bb);
  }
  sync();
  return dInput;
}

// Shared body of BackpropLinearProjection / BackpropOutputProjection
// (AccelerationCPU.cs:2188-2270): wgrad += dy^T x, bgrad += column sums of
// dy, dx (+)= dy w, over `rows` rows of x and dy.
void HipAccelerationManager::linear_backward(MatView x, MatView dy, int rows, MatView w,
                                             MatRef wgrad, VecRef bgrad, float *dx_host,
                                             bool accumulate_dx) {
  const int in = w.cols, out = w.rows;
  if (rows == 0 || in == 0) return;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t xb = (size_t)rows * in * sizeof(float), yb = (size_t)rows * out * sizeof(float);
  const size_t wb = (size_t)out * in * sizeof(float), bb = (size_t)out * sizeof(float);
  const float *dw = resident(w.data, out, in);
  float *dxin = static_cast<float *>(scratch(S_X, xb));
  float *ddy = static_cast<float *>(scratch(S_Q, yb > 0 ? yb : 4));
  float *ddx = static_cast<float *>(scratch(S_O, xb));
  float *gw = static_cast<float *>(scratch(S_GW0, wb > 0 ? wb : 4));
  float *gb = static_cast<float *>(scratch(S_GB0, bb > 0 ? bb : 4));
  upload(dxin, x.data, xb);
  if (out > 0) {
    upload(ddy, dy.data, yb);
    upload(gw, wgrad.data, wb);
    upload(gb, bgrad.data, bb);
  }
  if (accumulate_dx) upload(ddx, dx_host, xb);
  if (out > 0) {
    size_t ws = 0;
    check(cdml_linear_backward_workspace_size(rows, in, out, &ws),
          "cdml_linear_backward_workspace_size");
    void *dws = ws ? scratch(S_WS, ws) : nullptr;
    check(cdml_linear_backward(dxin, in, ddy, out, dw, ddx, in, gw, gb, rows, in, out,
                               accumulate_dx ? 1 : 0, dws, ws, stream_),
          "cdml_linear_backward");
  } else if (!accumulate_dx) {
    check(cdml_zero_f32_async(ddx, (size_t)rows * in, stream_), "cdml_zero_f32_async");
  }
  download(dx_host, ddx, xb);
  if (out > 0) {
    download(wgrad.data, gw, wb);
    download(bgrad.data, gb, bb);
  }
  sync();
}

// ---- BackpropLinearProjection: AccelerationCPU.cs:2188-2227 -----------------
// The reference indexes the arrays without checks (a mismatch surfaces as an
// IndexOutOfRangeException mid-update); here every shape is checked before
// any device work, with ArgumentException.
void HipAccelerationManager::BackpropLinearProjection(MatView input, MatView dOutput,
                                                      MatView weights, MatRef weightGrad,
                                                      VecRef biasGrad, MatRef dInput) {
  if (input.null()) throw ArgumentNullException("input");
  if (dOutput.null()) throw ArgumentNullException("dOutput");
  if (weights.null()) throw ArgumentNullException("weights");
  if (!weightGrad.data) throw ArgumentNullException("weightGrad");
  if (biasGrad.null()) throw ArgumentNullException("biasGrad");
  if (!dInput.data) throw ArgumentNullException("dInput");
  const int rows = input.rows, in = input.cols, out = dOutput.cols;
  if (dOutput.rows != rows) throw ArgumentException("dOutput rows must match input rows.", "dOutput");
  if (weights.rows != out || weights.cols != in)
    throw ArgumentException("weights must be [outDim, inDim].", "weights");
  if (weightGrad.rows != out || weightGrad.cols != in)
    throw ArgumentException("weightGrad must be [outDim, inDim].", "weightGrad");
  if (biasGrad.length != out) throw ArgumentException("biasGrad length must match outDim.", "biasGrad");
  if (dInput.rows != rows || dInput.cols != in)
    throw ArgumentException("dInput must be [seqLen, inDim].", "dInput");
  linear_backward(input, dOutput, rows, weights, weightGrad, biasGrad, dInput.data, true);
}

// ---- BackpropOutputProjection: AccelerationCPU.cs:2229-2270 ------------------
Matrix HipAccelerationManager::BackpropOutputProjection(MatView dLogits, MatView input,
                                                        MatView weights, MatRef weightGrad,
                                                        VecRef biasGrad, int seqLen, int outputDim,
                                                        int embeddingDim) {
  if (dLogits.null()) throw ArgumentNullException("dLogits");
  if (input.null()) throw ArgumentNullException("input");
  if (weights.null()) throw ArgumentNullException("weights");
  if (!weightGrad.data) throw ArgumentNullException("weightGrad");
  if (biasGrad.null()) throw ArgumentNullException("biasGrad");
  if (seqLen < 0 || seqLen > dLogits.rows || seqLen > input.rows)
    throw ArgumentException("seqLen exceeds the dLogits or input rows.", "seqLen");
  if (outputDim < 0 || dLogits.cols != outputDim)
    throw ArgumentException("dLogits width must equal outputDim.", "outputDim");
  if (embeddingDim < 0 || input.cols != embeddingDim)
    throw ArgumentException("input width must equal embeddingDim.", "embeddingDim");
  if (weights.rows != outputDim || weights.cols != embeddingDim)
    throw ArgumentException("weights must be [outputDim, embeddingDim].", "weights");
  if (weightGrad.rows != outputDim || weightGrad.cols != embeddingDim)
    throw ArgumentException("weightGrad must be [outputDim, embeddingDim].", "weightGrad");
  if (biasGrad.length != outputDim) throw ArgumentException("biasGrad length must match outputDim.", "biasGrad");
  Matrix dX(seqLen, embeddingDim);
  linear_backward(input, dLogits, seqLen, weights, weightGrad, biasGrad, dX.ptr(), false);
  return dX;
}

// ---- MatrixMultiply / MatrixMultiplyTranspose: AccelerationCPU.cs:159-250 ----
Matrix HipAccelerationManager::MatrixMultiply(MatView A, MatView B) {
  if (A.null()) throw ArgumentNullException("A");
  if (B.null()) throw ArgumentNullException("B");
  if (A.cols != B.rows)
    throw ArgumentException("Matrix dimensions don't match: [" + std::to_string(A.rows) + "x" +
                            std::to_string(A.cols) + "] * [" + std::to_string(B.rows) + "x" +
                            std::to_string(B.cols) + "]");
  Matrix C(A.rows, B.cols);
  if (A.rows == 0 || B.cols == 0 || A.cols == 0) return C;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t ab = (size_t)A.rows * A.cols * 4, bb = (size_t)B.rows * B.cols * 4,
               cb = (size_t)A.rows * B.cols * 4;
  float *da = static_cast<float *>(scratch(S_X, ab));
  float *db = static_cast<float *>(scratch(S_Q, bb));
  float *dc = static_cast<float *>(scratch(S_O, cb));
  upload(da, A.data, ab);
  upload(db, B.data, bb);
  check(cdml_matmul(da, A.cols, db, B.cols, dc, B.cols, A.rows, A.cols, B.cols, stream_), "cdml_matmul");
  download(C.ptr(), dc, cb);
  sync();
  return C;
}

Matrix HipAccelerationManager::MatrixMultiplyTranspose(MatView A, MatView B) {
  if (A.null()) throw ArgumentNullException("A");
  if (B.null()) throw ArgumentNullException("B");
  if (A.cols != B.cols) throw ArgumentException("Matrix dimensions don't match for A*B^T");
  Matrix C(A.rows, B.rows);
  if (A.rows == 0 || B.rows == 0 || A.cols == 0) return C;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t ab = (size_t)A.rows * A.cols * 4, bb = (size_t)B.rows * B.cols * 4,
               cb = (size_t)A.rows * B.rows * 4;
  float *da = static_cast<float *>(scratch(S_X, ab));
  float *db = static_cast<float *>(scratch(S_Q, bb));
  float *dc = static_cast<float *>(scratch(S_O, cb));
  upload(da, A.data, ab);
  upload(db, B.data, bb);
  check(cdml_linear(da, A.cols, db, nullptr, dc, B.rows, A.rows, A.cols, B.rows, CDML_ACT_NONE, stream_),
        "cdml_linear");
  download(C.ptr(), dc, cb);
  sync();
  return C;
}

// ---- ResidualLayerNormForward: AccelerationCPU.cs:1440-1514 -------------------
std::tuple<Matrix, std::vector<float>, std::vector<float>, Matrix, Matrix>
HipAccelerationManager::ResidualLayerNormForward(MatView input, MatView subLayer, VecView gamma,
                                                 VecView beta, float epsilon) {
  if (input.null()) throw ArgumentNullException("input");
  if (subLayer.null()) throw ArgumentNullException("subLayer");
  if (gamma.null()) throw ArgumentNullException("gamma");
  if (beta.null()) throw ArgumentNullException("beta");
  const int rows = input.rows, f = input.cols;
  if (subLayer.rows != rows || subLayer.cols != f)
    throw ArgumentException("Residual input dimensions must match.", "subLayer");
  if (gamma.length != f || beta.length != f)
    throw ArgumentException("Layer norm gamma/beta must match the feature dimension.");
  if (f > 2048) throw ArgumentException("ResidualLayerNormForward supports up to 2048 features.", "input");
  Matrix out(rows, f), norm(rows, f), res(rows, f);
  std::vector<float> mean(rows), var(rows);
  if (rows == 0 || f == 0) return {std::move(out), std::move(mean), std::move(var), std::move(norm), std::move(res)};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t bytes = (size_t)rows * f * 4;
  const float *dg = resident(gamma.data, 1, f), *dbt = resident(beta.data, 1, f);
  float *da = static_cast<float *>(scratch(S_X, bytes));
  float *dbb = static_cast<float *>(scratch(S_Q, bytes));
  float *dy = static_cast<float *>(scratch(S_O, bytes));
  float *dn = static_cast<float *>(scratch(S_K, bytes));
  float *dr = static_cast<float *>(scratch(S_V, bytes));
  float *dm = static_cast<float *>(scratch(S_DQ, (size_t)rows * 8));
  upload(da, input.data, bytes);
  upload(dbb, subLayer.data, bytes);
  check(cdml_residual_layernorm_fwd(da, dbb, dg, dbt, dy, dm, dm + rows, dr, dn, rows, f, epsilon, stream_),
        "cdml_residual_layernorm_fwd");
  download(out.ptr(), dy, bytes);
  download(norm.ptr(), dn, bytes);
  download(res.ptr(), dr, bytes);
  download(mean.data(), dm, (size_t)rows * 4);
  download(var.data(), dm + rows, (size_t)rows * 4);
  sync();
  return {std::move(out), std::move(mean), std::move(var), std::move(norm), std::move(res)};
}

// ---- LayerNormBackward: AccelerationCPU.cs:1516-1564 ----------------------------
// The reference indexes its arguments without checks; every shape is checked
// here first (ArgumentException).
std::tuple<Matrix, std::vector<float>, std::vector<float>>
HipAccelerationManager::LayerNormBackward(MatView dOut, MatView normalized, VecView gamma, MatView input,
                                          VecView mean, VecView variance, float epsilon) {
  if (dOut.null()) throw ArgumentNullException("dOut");
  if (normalized.null()) throw ArgumentNullException("normalized");
  if (gamma.null()) throw ArgumentNullException("gamma");
  if (input.null()) throw ArgumentNullException("input");
  if (mean.null()) throw ArgumentNullException("mean");
  if (variance.null()) throw ArgumentNullException("variance");
  const int rows = dOut.rows, f = dOut.cols;
  if (normalized.rows != rows || normalized.cols != f || input.rows != rows || input.cols != f)
    throw ArgumentException("normalized and input must have dOut's shape.");
  if (gamma.length != f) throw ArgumentException("gamma must match the feature dimension.", "gamma");
  if (mean.length < rows || variance.length < rows)
    throw ArgumentException("mean and variance need one entry per row.");
  if (f > 2048) throw ArgumentException("LayerNormBackward supports up to 2048 features.", "dOut");
  Matrix dx(rows, f);
  std::vector<float> dg(f), db(f);
  if (rows == 0 || f == 0) return {std::move(dx), std::move(dg), std::move(db)};
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t bytes = (size_t)rows * f * 4;
  float *dd = static_cast<float *>(scratch(S_X, bytes));
  float *dn = static_cast<float *>(scratch(S_Q, bytes));
  float *di = static_cast<float *>(scratch(S_K, bytes));
  float *dxo = static_cast<float *>(scratch(S_O, bytes));
  float *dmv = static_cast<float *>(scratch(S_DQ, (size_t)rows * 8));
  float *dgb = static_cast<float *>(scratch(S_GB0, (size_t)f * 8 + 4 * (size_t)f));
  float *dgam = dgb + 2 * (size_t)f;
  size_t ws = 0;
  check(cdml_layernorm_backward_workspace_size(rows, f, &ws), "cdml_layernorm_backward_workspace_size");
  void *dws = scratch(S_WS, ws);
  upload(dd, dOut.data, bytes);
  upload(dn, normalized.data, bytes);
  upload(di, input.data, bytes);
  upload(dmv, mean.data, (size_t)rows * 4);
  upload(dmv + rows, variance.data, (size_t)rows * 4);
  upload(dgam, gamma.data, (size_t)f * 4);
  check(cdml_layernorm_backward(dd, nullptr, dn, dgam, di, dmv, dmv + rows, dxo, dgb, dgb + f, rows, f, epsilon,
                                0, dws, ws, stream_),
        "cdml_layernorm_backward");
  download(dx.ptr(), dxo, bytes);
  download(dg.data(), dgb, (size_t)f * 4);
  download(db.data(), dgb + f, (size_t)f * 4);
  sync();
  return {std::move(dx), std::move(dg), std::move(db)};
}

// ---- CrossEntropyLossAndGradient: AccelerationCPU.cs:2372-2440 -----------------
std::pair<float, Matrix> HipAccelerationManager::CrossEntropyLossAndGradient(
    MatView logits, const std::vector<int> &targets, int targetStart, int effectiveLen) {
  if (logits.null()) throw ArgumentNullException("logits");
  if (targetStart < 0 || effectiveLen < 0 || (long long)targetStart + effectiveLen > (long long)targets.size())
    throw ArgumentOutOfRangeException("targetStart");
  const int rows = logits.rows, v = logits.cols;
  Matrix dl(rows, v);
  if (effectiveLen == 0) return {0.f, std::move(dl)};
  // the reference reads row i < effectiveLen and the target's column without
  // checks; both are checked here
  if (effectiveLen > rows) throw ArgumentException("effectiveLen exceeds the logits rows.", "effectiveLen");
  for (int i = 0; i < effectiveLen; ++i)
    if ((unsigned)targets[targetStart + i] >= (unsigned)v)
      throw ArgumentOutOfRangeException("targets", "Target out of range: " + std::to_string(targets[targetStart + i]));
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t bytes = (size_t)rows * v * 4;
  float *dlog = static_cast<float *>(scratch(S_X, bytes));
  int *dt = static_cast<int *>(scratch(S_IDS, (size_t)effectiveLen * 4));
  float *dloss = static_cast<float *>(scratch(S_BIAS, 4));
  size_t ws = 0;
  check(cdml_cross_entropy_workspace_size(rows, &ws), "cdml_cross_entropy_workspace_size");
  void *dws = scratch(S_WS, ws);
  upload(dlog, logits.data, bytes);
  upload(dt, targets.data() + targetStart, (size_t)effectiveLen * 4);
  check(cdml_cross_entropy(dlog, v, dt, rows, v, effectiveLen, 1.0f, 1.0f, dloss, dlog, v, dws, ws, stream_),
        "cdml_cross_entropy");
  float loss = 0.f;
  download(dl.ptr(), dlog, bytes);
  download(&loss, dloss, 4);
  sync();
  return {loss, std::move(dl)};
}

// ---- MSELossAndGradient: AccelerationCPU.cs:2442-2490 -------------------------
std::pair<float, Matrix> HipAccelerationManager::MSELossAndGradient(MatView predictions, MatView targets,
                                                                    int targetStart, int effectiveLen) {
  if (predictions.null()) throw ArgumentNullException("predictions");
  if (targets.null()) throw ArgumentNullException("targets");
  const int rows = predictions.rows, o = predictions.cols;
  if (targetStart < 0 || effectiveLen < 0 || (long long)targetStart + effectiveLen > targets.rows || targets.cols != o)
    throw ArgumentException("Target shape must match predictions for the effective length and target offset.",
                            "targets");
  Matrix d(rows, o);
  if (effectiveLen == 0 || o == 0) return {0.f, std::move(d)};
  // the reference reads prediction rows i < effectiveLen without a check
  if (effectiveLen > rows) throw ArgumentException("effectiveLen exceeds the prediction rows.", "effectiveLen");
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t pbytes = (size_t)rows * o * 4, tbytes = (size_t)effectiveLen * o * 4;
  float *dp = static_cast<float *>(scratch(S_X, pbytes));
  float *dt = static_cast<float *>(scratch(S_Q, tbytes));
  float *dd = static_cast<float *>(scratch(S_K, pbytes));
  float *dloss = static_cast<float *>(scratch(S_BIAS, 4));
  void *dws = scratch(S_WS, (size_t)rows * 4);
  upload(dp, predictions.data, pbytes);
  upload(dt, targets.data + (size_t)targetStart * o, tbytes);
  check(cdml_mse_loss(dp, o, dt, o, rows, o, effectiveLen, 1.0f, 1.0f, dloss, dd, o, dws, (size_t)rows * 4, stream_),
        "cdml_mse_loss");
  float loss = 0.f;
  download(d.ptr(), dd, pbytes);
  download(&loss, dloss, 4);
  sync();
  return {loss, std::move(d)};
}

// ---- AccumulateTokenEmbeddingGrad: AccelerationCPU.cs:2339-2370 ----------------
void HipAccelerationManager::AccumulateTokenEmbeddingGrad(MatRef embeddingGrad, MatView dX,
                                                          const std::vector<int> &tokenIds, int tokenStart,
                                                          int seqLen, int embeddingDim) {
  if (!embeddingGrad.data) throw ArgumentNullException("embeddingGrad");
  if (dX.null()) throw ArgumentNullException("dX");
  if (tokenStart < 0 || seqLen < 0 || (long long)tokenStart + seqLen > (long long)tokenIds.size())
    throw ArgumentOutOfRangeException("tokenStart");
  if (embeddingGrad.cols != embeddingDim || dX.cols != embeddingDim || dX.rows < seqLen)
    throw ArgumentException("embeddingGrad and dX must be [*, embeddingDim] with seqLen rows of dX.");
  const int vocab = embeddingGrad.rows;
  for (int i = 0; i < seqLen; ++i)
    if ((unsigned)tokenIds[tokenStart + i] >= (unsigned)vocab)
      throw ArgumentOutOfRangeException("tokenIds", "Token out of range: " + std::to_string(tokenIds[tokenStart + i]));
  if (seqLen == 0 || embeddingDim == 0) return;
  // rows grouped by token, each group in row order (the reference's summation order)
  std::vector<int> order(seqLen);
  for (int i = 0; i < seqLen; ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return tokenIds[tokenStart + a] < tokenIds[tokenStart + b]; });
  std::vector<int> start, token;
  for (int i = 0; i < seqLen; ++i)
    if (i == 0 || tokenIds[tokenStart + order[i]] != tokenIds[tokenStart + order[i - 1]]) {
      start.push_back(i);
      token.push_back(tokenIds[tokenStart + order[i]]);
    }
  start.push_back(seqLen);
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t gb = (size_t)vocab * embeddingDim * 4, xb = (size_t)seqLen * embeddingDim * 4;
  float *dg = static_cast<float *>(scratch(S_O, gb));
  float *dx = static_cast<float *>(scratch(S_X, xb));
  int *di = static_cast<int *>(scratch(S_IDS, ((size_t)seqLen * 3 + 1) * 4));
  upload(dg, embeddingGrad.data, gb);
  upload(dx, dX.data, xb);
  upload(di, order.data(), (size_t)seqLen * 4);
  upload(di + seqLen, start.data(), start.size() * 4);
  upload(di + 2 * seqLen + 1, token.data(), token.size() * 4);
  check(cdml_embedding_grad(dg, dx, nullptr, embeddingDim, di, di + seqLen, di + 2 * seqLen + 1,
                            (int)token.size(), embeddingDim, stream_),
        "cdml_embedding_grad");
  download(embeddingGrad.data, dg, gb);
  sync();
}

// ---- decode capability ------------------------------------------------------
Matrix HipAccelerationManager::DecodeSelfAttention(MatRef q, MatRef k, MatView v, MatRef keys,
                                                   MatRef values, int absolutePosition,
                                                   int numHeads) {
  if (!q.data) throw ArgumentNullException("q");
  if (!k.data) throw ArgumentNullException("k");
  if (v.null()) throw ArgumentNullException("v");
  if (!keys.data) throw ArgumentNullException("keys");
  if (!values.data) throw ArgumentNullException("values");
  if (q.rows != 1 || k.rows != 1 || v.rows != 1)
    throw ArgumentException("Incremental RoPE expects single-row Q and K matrices.");
  const int dim = q.cols;
  if (k.cols != dim || v.cols != dim) throw ArgumentException("Q and K must have the same embedding dimension.");
  if (numHeads <= 0 || dim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by number of heads.", "numHeads");
  const int headDim = dim / numHeads;
  if (headDim & 1) throw ArgumentException("RoPE requires an even per-head dimension.");
  if (keys.cols != dim || values.cols != dim || values.rows != keys.rows)
    throw ArgumentException("Key/value caches must be [maxSeq, D] with D the query width.");
  if (absolutePosition < 0 || absolutePosition >= keys.rows)
    throw InvalidOperationException("Decoder KV cache is full.");
  Matrix out(1, dim);
  if (dim == 0) return out;
  std::lock_guard<std::mutex> lock(mu_);
  ensure_ready();
  const size_t row = (size_t)dim * sizeof(float);
  DecodeMirror &m = decode_[keys.data];
  if (m.rows != keys.rows || m.cols != dim) {
    sync();
    cdml_free(m.k);
    cdml_free(m.v);
    m = DecodeMirror{};
    check(cdml_malloc(&m.k, keys.rows * row), "cdml_malloc");
    check(cdml_malloc(&m.v, keys.rows * row), "cdml_malloc");
    m.rows = keys.rows;
    m.cols = dim;
  }
  if (m.uploaded != absolutePosition) {  // not the rows this manager appended: refresh
    upload(m.k, keys.data, (size_t)absolutePosition * row);
    upload(m.v, values.data, (size_t)absolutePosition * row);
  }
  float *dq = static_cast<float *>(scratch(S_Q, row));
  float *dout = static_cast<float *>(scratch(S_O, row));
  int *dlen = static_cast<int *>(scratch(S_KVLEN, sizeof(int)));
  float *dk = static_cast<float *>(m.k) + (size_t)absolutePosition * dim;
  float *dv = static_cast<float *>(m.v) + (size_t)absolutePosition * dim;
  size_t ws = 0;
  check(cdml_decode_attn_workspace_size(1, keys.rows, dim, numHeads, &ws),
        "cdml_decode_attn_workspace_size");
  void *dws = scratch(S_WS, ws);
  upload(dq, q.data, row);
  upload(dk, k.data, row);
  upload(dv, v.data, row);
  check(cdml_rope(dq, 1, dim, 0, headDim, numHeads, 10000.0f, 0, absolutePosition, 0, nullptr, stream_),
        "cdml_rope");
  check(cdml_rope(dk, 1, dim, 0, headDim, numHeads, 10000.0f, 0, absolutePosition, 0, nullptr, stream_),
        "cdml_rope");
  check(cdml_fill_i32_async(dlen, 1, absolutePosition + 1, stream_), "cdml_fill_i32_async");
  const float scale = 1.0f / std::sqrt((float)headDim);  // LanguageModel.cs:368
  check(cdml_decode_attn(dq, static_cast<const float *>(m.k), static_cast<const float *>(m.v), dlen,
                         dout, 1, keys.rows, dim, numHeads, scale, dws, ws, stream_),
        "cdml_decode_attn");
  download(q.data, dq, row);
  download(k.data, dk, row);
  download(out.ptr(), dout, row);
  sync();
  m.uploaded = absolutePosition + 1;
  std::memcpy(keys.data + (size_t)absolutePosition * dim, k.data, row);
  std::memcpy(values.data + (size_t)absolutePosition * dim, v.data, row);
  return out;
}

}  // namespace cdml_host
