// The decoder-only model of Transformers/MultiTypeTransformer restated over
// HipAccelerationManager (MultiHeadAttention, TransformerBlock,
// LanguageModel), and DeviceLanguageModel, the device-resident engine for the
// same weights.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "cdml_host.h"

namespace cdml_host {

namespace {

void check(int rc, const char *what) {
  if (rc != CDML_OK)
    throw InvalidOperationException(std::string(what) + ": " + cdml_last_error());
}

// SplitMix64 (Steele, Lea, Flood 2014): the sampler's random stream.
uint64_t splitmix64(uint64_t &s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

// ---- TransformerConfig.Validate: TransformerConfig.cs:62-102 ---------------
// TransformerConfig.Validate (TransformerConfig.cs:61-101) in the reference's
// order: the module base (SharedConfigs.cs:150-157), the sizes, then
// DataConfig / RuntimeConfig / RegularizationConfig (DataConfig.cs:30-40,
// SharedConfigs.cs:239-254,266-270), then the attention rules.  Positive-size
// and enum checks throw ArgumentException, as ConfigBase.RequirePositive does
// (ConfigBase.cs:16-54).
void TransformerConfig::Validate() const {
  auto positive = [](int v, const char *n) {
    if (v <= 0) throw ArgumentException(std::string(n) + " must be positive, got " + std::to_string(v) + ".");
  };
  auto fmt = [](float v) {
    char b[32];
    std::snprintf(b, sizeof b, "%g", (double)v);
    return std::string(b);
  };
  positive(EmbeddingDim, "EmbeddingDim");
  positive(NumHeads, "NumHeads");
  positive(NumLayers, "NumLayers");
  positive(FeedForwardDim, "FeedForwardDim");
  if (EmbeddingDim % NumHeads != 0)
    throw ArgumentException("EmbeddingDim (" + std::to_string(EmbeddingDim) +
                                ") must be divisible by NumHeads (" + std::to_string(NumHeads) + ").",
                            "EmbeddingDim");
  positive(VocabSize, "VocabSize");
  positive(MaxSequenceLength, "MaxSequenceLength");
  positive(InputFeatureDim, "InputFeatureDim");
  positive(OutputDim, "OutputDim");
  if (DataType < 0 || DataType > 3) throw ArgumentException("Invalid DataType: " + std::to_string(DataType) + ".");
  if (CostFunction < 0 || CostFunction > 5)
    throw ArgumentException("Invalid CostFunction: " + std::to_string(CostFunction) + ".");
  if (ActivationDistribution < 0 || ActivationDistribution > 1)
    throw ArgumentException("Invalid ActivationDistribution: " + std::to_string(ActivationDistribution) + ".");
  if (FFNActivationType < None || FFNActivationType > Swish)
    throw ArgumentException("Invalid FFNActivationType value: " + std::to_string(FFNActivationType) + ".");
  if (AccelerationType < 0 || AccelerationType > 4)
    throw ArgumentException("Invalid AccelerationType value: " + std::to_string(AccelerationType) + ".");
  if (AccelerationDeviceId < 0)
    throw ArgumentException("AccelerationDeviceId must be non-negative, got " +
                            std::to_string(AccelerationDeviceId) + ".");
  if (!(L2RegulationLamda >= 0.f))
    throw ArgumentException("L2RegulationLamda must be non-negative, got " + fmt(L2RegulationLamda) + ".");
  if (!(GradientClippingThreshold > 0.f))
    throw ArgumentException("GradientClippingThreshold must be positive, got " + fmt(GradientClippingThreshold) + ".");
  if ((EmbeddingDim / NumHeads) & 1)
    throw ArgumentException("RoPE requires an even per-head dimension. EmbeddingDim / NumHeads = " +
                                std::to_string(EmbeddingDim / NumHeads) + ".",
                            "EmbeddingDim");
  if (UsesDiscreteTokens) {
    if (VocabSize < 2) throw ArgumentException("Discrete token models require VocabSize >= 2.", "VocabSize");
  } else if (DataType == 2 && OutputDim < 2) {
    throw ArgumentException("TimeSeriesClassification requires OutputDim >= 2 classes.", "OutputDim");
  }
}

// ---- MultiHeadAttention: MultiHeadAttention.cs:23-159 ------------------------
MultiHeadAttention::MultiHeadAttention(int embeddingDim, int numHeads, HipAccelerationManager *accel)
    : dim_(embeddingDim), heads_(numHeads), accel_(accel) {
  if (embeddingDim <= 0) throw ArgumentOutOfRangeException("embeddingDim", "Embedding dimension must be positive.");
  if (numHeads <= 0) throw ArgumentOutOfRangeException("numHeads", "Number of heads must be positive.");
  if (embeddingDim % numHeads != 0)
    throw ArgumentException("Embedding dimension must be divisible by number of heads.", "numHeads");
  head_dim_ = embeddingDim / numHeads;
  if (head_dim_ & 1) throw ArgumentException("RoPE requires an even per-head dimension.", "embeddingDim");
  if (!accel) throw ArgumentNullException("accel");
  // Weights are set by the owner (the reference draws them from System.Random,
  // MultiHeadAttention.cs:63-89, which is not reproduced); biases start at 0.
  WQ = Matrix(dim_, dim_);
  WK = Matrix(dim_, dim_);
  WV = Matrix(dim_, dim_);
  WO = Matrix(dim_, dim_);
  BiasQ.assign(dim_, 0.f);
  BiasK.assign(dim_, 0.f);
  BiasV.assign(dim_, 0.f);
  BiasO.assign(dim_, 0.f);
}

Matrix MultiHeadAttention::Forward(MatView input, MaskView mask, bool causal) {
  if (input.null()) throw ArgumentNullException("input");
  if (input.cols != dim_)
    throw ArgumentException("Input width must be " + std::to_string(dim_) + ".", "input");
  if (input.rows <= 0) throw ArgumentException("Sequence must contain at least one row.", "input");
  if (!mask.null() && (mask.rows != input.rows || mask.cols != input.rows))
    throw ArgumentException("Mask shape must match the sequence length.", "mask");
  auto qkv = accel_->ProjectQKV(input, WQ, BiasQ, WK, BiasK, WV, BiasV);
  Matrix &Q = std::get<0>(qkv), &K = std::get<1>(qkv), &V = std::get<2>(qkv);
  // RotaryPositionEmbedding.ApplyInPlace(Q, K, numHeads): RotaryPositionEmbedding.cs:20-73
  accel_->ApplyRotaryPositionEmbeddingInPlace(Q, heads_, 10000.0f, false);
  accel_->ApplyRotaryPositionEmbeddingInPlace(K, heads_, 10000.0f, false);
  Matrix concatenated = accel_->ScaledDotProductAttention(Q, K, V, heads_, mask, causal);
  return accel_->ProjectOutputBatch(concatenated, WO, BiasO, concatenated.rows, dim_);
}

// ---- TransformerBlock: TransformerBlock.cs:35-62, 79-129 ----------------------
TransformerBlock::TransformerBlock(int embeddingDim, int numHeads, int feedForwardDim,
                                   int ffnActivation, HipAccelerationManager *accel)
    : Attention(embeddingDim, numHeads, accel), accel_(accel) {
  LN1Gamma.assign(embeddingDim, 1.f);
  LN1Beta.assign(embeddingDim, 0.f);
  LN2Gamma.assign(embeddingDim, 1.f);
  LN2Beta.assign(embeddingDim, 0.f);
  // widths [D, FF, D], activations [None, act, None]: the hidden layer takes
  // the configured activation, the output layer none.
  FeedForward.weights = {Matrix(feedForwardDim, embeddingDim), Matrix(embeddingDim, feedForwardDim)};
  FeedForward.biases = {std::vector<float>(feedForwardDim, 0.f), std::vector<float>(embeddingDim, 0.f)};
  FeedForward.activations = {ffnActivation, None};
}

Matrix TransformerBlock::Forward(MatView x, MaskView selfMask, bool causal) {
  Matrix selfOut = Attention.Forward(x, selfMask, causal);
  Matrix normedSelf = accel_->ResidualLayerNorm(x, selfOut, LN1Gamma, LN1Beta);
  // CrossAttentionForward is the identity for the plain block (:131-136).
  Matrix ffOut = accel_->FFNForwardBatch(normedSelf, normedSelf.rows, normedSelf.cols, FeedForward);
  return accel_->ResidualLayerNorm(normedSelf, ffOut, LN2Gamma, LN2Beta);
}

// ---- LanguageModel: LanguageModel.cs ------------------------------------------
LanguageModel::LanguageModel(const TransformerConfig &cfg, HipAccelerationManager *accel)
    : cfg_(cfg), accel_(accel) {
  cfg_.Validate();
  if (!accel) throw ArgumentNullException("accel");
  const int D = cfg_.EmbeddingDim;
  if (cfg_.UsesDiscreteTokens) {
    TokenEmbedding = Matrix(cfg_.VocabSize, D);
  } else {
    InputProjection = Matrix(D, cfg_.InputFeatureDim);
    InputProjectionBias.assign(D, 0.f);
  }
  OutputProjection = Matrix(cfg_.EffectiveOutputDim(), D);
  OutputBias.assign(cfg_.EffectiveOutputDim(), 0.f);
  Blocks.reserve(cfg_.NumLayers);
  for (int i = 0; i < cfg_.NumLayers; ++i)
    Blocks.emplace_back(D, cfg_.NumHeads, cfg_.FeedForwardDim, cfg_.FFNActivationType, accel);
}

// :585-600
void LanguageModel::ValidateTokenSequence(const std::vector<int> &ids) const {
  if (ids.empty()) throw ArgumentException("Token sequence must contain at least one token.", "tokenIds");
  if ((int)ids.size() > cfg_.MaxSequenceLength)
    throw ArgumentException("Token sequence length " + std::to_string(ids.size()) +
                                " exceeds MaxSequenceLength " +
                                std::to_string(cfg_.MaxSequenceLength) + ".",
                            "tokenIds");
  for (size_t i = 0; i < ids.size(); ++i)
    if ((unsigned)ids[i] >= (unsigned)cfg_.VocabSize)
      throw ArgumentOutOfRangeException("tokenIds", "Token id " + std::to_string(ids[i]) +
                                                        " at position " + std::to_string(i) +
                                                        " is outside [0, " +
                                                        std::to_string(cfg_.VocabSize) + ").");
}

// :210-223: causal = UseDecoderOnly, no mask
Matrix LanguageModel::ForwardHidden(Matrix x) {
  for (auto &block : Blocks) x = block.Forward(x, MaskView{}, cfg_.UseDecoderOnly);
  return x;
}

// :225-233
Matrix LanguageModel::ProjectToOutput(const Matrix &hidden) {
  return accel_->ProjectOutputBatch(hidden, OutputProjection, OutputBias, hidden.rows,
                                    cfg_.EffectiveOutputDim());
}

// :112-122
Matrix LanguageModel::Forward(const std::vector<int> &tokenIds) {
  if (!cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Use Forward(float[,]) for continuous input data types.");
  ValidateTokenSequence(tokenIds);
  Matrix embedded = accel_->EmbedTokenIds(tokenIds, TokenEmbedding, cfg_.EmbeddingDim);
  return ProjectToOutput(ForwardHidden(std::move(embedded)));
}

// :124-133 (EmbedContinuous = BatchDotProductAddBias(InputProjection, x, bias), :186-189)
Matrix LanguageModel::Forward(MatView inputSequence) {
  if (cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Use Forward(int[]) for discrete token data types.");
  if (inputSequence.null()) throw ArgumentNullException("inputSequence");
  if (inputSequence.rows <= 0 || inputSequence.rows > cfg_.MaxSequenceLength)
    throw ArgumentException("Sequence length must be in [1, MaxSequenceLength].", "inputSequence");
  if (inputSequence.cols != cfg_.InputFeatureDim)
    throw ArgumentException("Input width must equal InputFeatureDim.", "inputSequence");
  Matrix embedded = accel_->BatchDotProductAddBias(InputProjection, inputSequence, InputProjectionBias);
  return ProjectToOutput(ForwardHidden(std::move(embedded)));
}

// :135-144 with ValidateTokenSlice (:602-619)
Matrix LanguageModel::ForwardTokenSlice(const std::vector<int> &tokenIds, int tokenStart, int tokenCount) {
  if (!cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Use ForwardContinuousSlice(float[,], int, int) for continuous input data types.");
  if (tokenCount <= 0) throw ArgumentException("Token slice must contain at least one token.", "tokenCount");
  if (tokenStart < 0 || (long long)tokenStart + tokenCount > (long long)tokenIds.size())
    throw ArgumentOutOfRangeException("tokenStart");
  if (tokenCount > cfg_.MaxSequenceLength)
    throw ArgumentException("Token sequence length " + std::to_string(tokenCount) + " exceeds MaxSequenceLength " +
                                std::to_string(cfg_.MaxSequenceLength) + ".",
                            "tokenCount");
  for (int i = 0; i < tokenCount; ++i) {
    const int token = tokenIds[tokenStart + i];
    if ((unsigned)token >= (unsigned)cfg_.VocabSize)
      throw ArgumentOutOfRangeException("tokenIds", "Token id " + std::to_string(token) + " at position " +
                                                        std::to_string(tokenStart + i) + " is outside [0, " +
                                                        std::to_string(cfg_.VocabSize) + ").");
  }
  Matrix embedded = accel_->EmbedTokenIds(tokenIds, tokenStart, tokenCount, TokenEmbedding, cfg_.EmbeddingDim);
  return ProjectToOutput(ForwardHidden(std::move(embedded)));
}

// :146-157 with ValidateContinuousSlice (:642-668)
Matrix LanguageModel::ForwardContinuousSlice(MatView inputSequence, int rowStart, int rowCount) {
  if (cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Use ForwardTokenSlice(int[], int, int) for discrete token data types.");
  if (inputSequence.null()) throw ArgumentNullException("inputSequence");
  if (rowCount <= 0) throw ArgumentException("Input sequence slice must contain at least one row.", "rowCount");
  if (rowStart < 0 || (long long)rowStart + rowCount > inputSequence.rows) throw ArgumentOutOfRangeException("rowStart");
  if (rowCount > cfg_.MaxSequenceLength)
    throw ArgumentException("Input sequence length " + std::to_string(rowCount) + " exceeds MaxSequenceLength " +
                                std::to_string(cfg_.MaxSequenceLength) + ".",
                            "rowCount");
  if (inputSequence.cols != cfg_.InputFeatureDim)
    throw ArgumentException("Input feature dimension must be " + std::to_string(cfg_.InputFeatureDim) + ", got " +
                                std::to_string(inputSequence.cols) + ".",
                            "inputSequence");
  for (int i = 0; i < rowCount; ++i)
    for (int j = 0; j < inputSequence.cols; ++j) {
      const float v = inputSequence.data[(size_t)(rowStart + i) * inputSequence.cols + j];
      if (std::isnan(v) || std::isinf(v))
        throw ArgumentException("Input value at [" + std::to_string(rowStart + i) + "," + std::to_string(j) +
                                    "] is not finite.",
                                "inputSequence");
    }
  Matrix embedded =
      accel_->BatchDotProductAddBias(InputProjection, inputSequence, rowStart, rowCount, InputProjectionBias);
  return ProjectToOutput(ForwardHidden(std::move(embedded)));
}

// :235-268, with the dot products on the device (the reference runs this
// inline on the host).
std::vector<float> LanguageModel::ProjectLastTokenOnly(const Matrix &hidden) {
  if (hidden.rows <= 0) throw ArgumentException("Hidden states must contain at least one row.", "hidden");
  MatView last(hidden.ptr() + (size_t)(hidden.rows - 1) * hidden.cols, 1, hidden.cols);
  Matrix logits = accel_->ProjectOutputBatch(last, OutputProjection, OutputBias, 1, cfg_.EffectiveOutputDim());
  return std::vector<float>(logits.data.begin(), logits.data.end());
}

// :602-612 (PredictNext)
std::vector<float> LanguageModel::PredictNext(MatView inputSequence) {
  if (cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Must use Generate() for discrete token data types.");
  if (inputSequence.null()) throw ArgumentNullException("inputSequence");
  Matrix embedded = accel_->BatchDotProductAddBias(InputProjection, inputSequence, InputProjectionBias);
  return ProjectLastTokenOnly(ForwardHidden(std::move(embedded)));
}

// :334-430, with the step's RoPE, cache append and attention on the
// manager's decode capability.
Matrix LanguageModel::DecoderSelfAttentionStep(MultiHeadAttention &attn, const Matrix &input,
                                               int absolutePosition, LayerCache &cache) {
  if (cache.Length != absolutePosition)
    throw InvalidOperationException("Decoder KV cache length " + std::to_string(cache.Length) +
                                    " does not match requested absolute position " +
                                    std::to_string(absolutePosition) + ".");
  if (cache.Length >= cfg_.MaxSequenceLength) throw InvalidOperationException("Decoder KV cache is full.");
  auto qkv = accel_->ProjectQKV(input, attn.WQ, attn.BiasQ, attn.WK, attn.BiasK, attn.WV, attn.BiasV);
  Matrix &q = std::get<0>(qkv), &k = std::get<1>(qkv), &v = std::get<2>(qkv);
  Matrix concatenated =
      accel_->DecodeSelfAttention(q, k, v, cache.Keys, cache.Values, absolutePosition, cfg_.NumHeads);
  cache.Length++;
  return accel_->ProjectOutputBatch(concatenated, attn.WO, attn.BiasO, 1, cfg_.EmbeddingDim);
}

// :294-332
Matrix LanguageModel::DecoderTokenStep(int tokenId, int absolutePosition, std::vector<LayerCache> &caches) {
  const int D = cfg_.EmbeddingDim;
  Matrix x(1, D);
  std::memcpy(x.ptr(), TokenEmbedding.ptr() + (size_t)tokenId * D, D * sizeof(float));
  for (int layer = 0; layer < cfg_.NumLayers; ++layer) {
    TransformerBlock &block = Blocks[layer];
    Matrix attnOut = DecoderSelfAttentionStep(block.Attention, x, absolutePosition, caches[layer]);
    Matrix normedSelf = accel_->ResidualLayerNorm(x, attnOut, block.LN1Gamma, block.LN1Beta);
    Matrix ffnOut = accel_->FFNForwardBatch(normedSelf, 1, D, block.FeedForward);
    x = accel_->ResidualLayerNorm(normedSelf, ffnOut, block.LN2Gamma, block.LN2Beta);
  }
  return x;
}

// Greedy: the lowest index holding the maximum.  Sampling: the reference's
// SampleFromLogits (:551-584) on logits / temperature with a SplitMix64 draw.
int LanguageModel::NextToken(const std::vector<float> &logits, float temperature, bool greedy,
                             uint64_t &rng_state) const {
  for (size_t i = 0; i < logits.size(); ++i)
    if (!std::isfinite(logits[i]))
      throw InvalidOperationException("Logit at index " + std::to_string(i) + " is not finite.");
  if (greedy) return (int)(std::max_element(logits.begin(), logits.end()) - logits.begin());
  float mx = -INFINITY;
  std::vector<float> l(logits.size());
  for (size_t i = 0; i < l.size(); ++i) {
    l[i] = logits[i] / temperature;
    mx = std::max(mx, l[i]);
  }
  float sum = 0.f;
  for (float x : l) sum += std::exp(x - mx);
  if (!(sum > 0.f) || std::isinf(sum))
    throw InvalidOperationException("Cannot sample because softmax normalization is invalid.");
  const float u = (float)((splitmix64(rng_state) >> 40) * (1.0 / (1ull << 24)));
  const float threshold = u * sum;
  float cumulative = 0.f;
  for (size_t i = 0; i < l.size(); ++i) {
    cumulative += std::exp(l[i] - mx);
    if (threshold < cumulative) return (int)i;
  }
  return (int)l.size() - 1;
}

// :482-537
std::vector<int> LanguageModel::Generate(const std::vector<int> &prompt, int maxNewTokens,
                                         float temperature, bool greedy, uint64_t seed) {
  if (!cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Generate is only supported for discrete token data types.");
  ValidateTokenSequence(prompt);
  if (maxNewTokens < 0) throw ArgumentOutOfRangeException("maxNewTokens", "maxNewTokens must be non-negative.");
  if (std::isnan(temperature) || std::isinf(temperature) || temperature <= 0.f)
    throw ArgumentOutOfRangeException("temperature", "temperature must be finite and greater than zero.");
  std::vector<int> tokens(prompt);
  if ((int)tokens.size() >= cfg_.MaxSequenceLength || maxNewTokens == 0) return tokens;
  uint64_t rng = seed;
  if (!cfg_.UseDecoderOnly) {
    for (int i = 0; i < maxNewTokens && (int)tokens.size() < cfg_.MaxSequenceLength; ++i) {
      Matrix hidden = ForwardHidden(accel_->EmbedTokenIds(tokens, TokenEmbedding, cfg_.EmbeddingDim));
      tokens.push_back(NextToken(ProjectLastTokenOnly(hidden), temperature, greedy, rng));
    }
    return tokens;
  }
  std::vector<LayerCache> caches(cfg_.NumLayers);
  for (auto &c : caches) {
    c.Keys = Matrix(cfg_.MaxSequenceLength, cfg_.EmbeddingDim);
    c.Values = Matrix(cfg_.MaxSequenceLength, cfg_.EmbeddingDim);
  }
  Matrix lastHidden;
  for (int pos = 0; pos < (int)tokens.size(); ++pos) lastHidden = DecoderTokenStep(tokens[pos], pos, caches);
  for (int generated = 0; generated < maxNewTokens && (int)tokens.size() < cfg_.MaxSequenceLength;
       ++generated) {
    const int next = NextToken(ProjectLastTokenOnly(lastHidden), temperature, greedy, rng);
    tokens.push_back(next);
    if ((int)tokens.size() < cfg_.MaxSequenceLength && generated + 1 < maxNewTokens)
      lastHidden = DecoderTokenStep(next, (int)tokens.size() - 1, caches);
  }
  return tokens;
}

// ---- DeviceLanguageModel -------------------------------------------------------
float *DeviceLanguageModel::alloc(size_t floats) {
  void *p = nullptr;
  check(cdml_malloc(&p, std::max<size_t>(floats, 1) * sizeof(float)), "cdml_malloc");
  allocs_.push_back(p);
  return static_cast<float *>(p);
}

float *DeviceLanguageModel::upload(const float *host, size_t floats) {
  float *d = alloc(floats);
  if (floats) check(cdml_memcpy_h2d_async(d, host, floats * sizeof(float), stream_), "cdml_memcpy_h2d_async");
  return d;
}

DeviceLanguageModel::DeviceLanguageModel(const LanguageModel &model, int batch_capacity, int device)
    : cfg_(model.config()), cap_(batch_capacity), device_(device) {
  if (batch_capacity <= 0) throw ArgumentOutOfRangeException("batch_capacity");
  check(cdml_init(device), "cdml_init");
  check(cdml_stream_create(&stream_), "cdml_stream_create");
  try {
    const int D = cfg_.EmbeddingDim, S = cfg_.MaxSequenceLength, O = cfg_.EffectiveOutputDim();
    const size_t rows = (size_t)cap_ * S;
    if (cfg_.UsesDiscreteTokens) {
      emb_ = upload(model.TokenEmbedding.ptr(), model.TokenEmbedding.data.size());
    } else {
      inproj_ = upload(model.InputProjection.ptr(), model.InputProjection.data.size());
      inbias_ = upload(model.InputProjectionBias.data(), model.InputProjectionBias.size());
    }
    outproj_ = upload(model.OutputProjection.ptr(), model.OutputProjection.data.size());
    outbias_ = upload(model.OutputBias.data(), model.OutputBias.size());
    ff_max_ = std::max(D, cfg_.UsesDiscreteTokens ? 0 : cfg_.InputFeatureDim);
    for (const auto &b : model.Blocks) {
      Layer L{};
      const MultiHeadAttention &a = b.Attention;
      L.wq = upload(a.WQ.ptr(), a.WQ.data.size());
      L.wk = upload(a.WK.ptr(), a.WK.data.size());
      L.wv = upload(a.WV.ptr(), a.WV.data.size());
      L.wo = upload(a.WO.ptr(), a.WO.data.size());
      L.bq = upload(a.BiasQ.data(), D);
      L.bk = upload(a.BiasK.data(), D);
      L.bv = upload(a.BiasV.data(), D);
      L.bo = upload(a.BiasO.data(), D);
      L.ln1g = upload(b.LN1Gamma.data(), D);
      L.ln1b = upload(b.LN1Beta.data(), D);
      L.ln2g = upload(b.LN2Gamma.data(), D);
      L.ln2b = upload(b.LN2Beta.data(), D);
      int width = D;
      for (size_t l = 0; l < b.FeedForward.weights.size(); ++l) {
        const Matrix &w = b.FeedForward.weights[l];
        if (w.cols != width) throw ArgumentException("FFN layer widths do not chain.");
        L.ffw.push_back(upload(w.ptr(), w.data.size()));
        L.ffb.push_back(upload(b.FeedForward.biases[l].data(), w.rows));
        L.ffrows.push_back(w.rows);
        L.ffcols.push_back(w.cols);
        L.ffact.push_back(b.FeedForward.activations[l]);
        ff_max_ = std::max(ff_max_, w.rows);
        width = w.rows;
      }
      if (width != D) throw ArgumentException("FFN output width must equal EmbeddingDim.");
      L.kcache = alloc(rows * D);
      L.vcache = alloc(rows * D);
      layers_.push_back(std::move(L));
    }
    x_ = alloc(rows * D);
    q_ = alloc(rows * D);
    k_ = alloc(rows * D);
    v_ = alloc(rows * D);
    att_ = alloc(rows * D);
    proj_ = alloc(rows * D);
    h_ = alloc(rows * D);
    ff_ = alloc(rows * ff_max_);
    ff2_ = alloc(rows * ff_max_);
    logits_ = alloc(rows * (size_t)O);
    ids_ = reinterpret_cast<int *>(alloc(rows));
    pos_ = reinterpret_cast<int *>(alloc(cap_));
    kvlen_ = reinterpret_cast<int *>(alloc(cap_));
    gen_ = reinterpret_cast<int *>(alloc(rows));
    check(cdml_decode_attn_workspace_size(cap_, S, D, cfg_.NumHeads, &ws_bytes_), "workspace size");
    ws_ = alloc(ws_bytes_ / sizeof(float) + 1);
    // (cos, sin) of every position the model can see, shared by all layers
    rope_cs_ = alloc((size_t)S * (D / cfg_.NumHeads));
    check(cdml_rope_table(rope_cs_, S, D / cfg_.NumHeads, 10000.0f, stream_), "cdml_rope_table");
    // descriptors of the fused decode path, when the model is within its limits
    if (cfg_.UsesDiscreteTokens && cfg_.UseDecoderOnly && D <= 256 && (D / cfg_.NumHeads) % 4 == 0 &&
        (long long)cfg_.NumHeads * S <= 4096) {
      std::vector<cdml_tiny_layer> tl(layers_.size());
      bool ok = true;
      for (size_t i = 0; i < layers_.size() && ok; ++i) {
        const Layer &L = layers_[i];
        cdml_tiny_layer &T = tl[i];
        T.wq = L.wq; T.bq = L.bq; T.wk = L.wk; T.bk = L.bk; T.wv = L.wv; T.bv = L.bv; T.wo = L.wo; T.bo = L.bo;
        T.ln1g = L.ln1g; T.ln1b = L.ln1b; T.ln2g = L.ln2g; T.ln2b = L.ln2b;
        T.n_ff = (int)L.ffw.size();
        if (T.n_ff > CDML_TINY_MAX_FF) {
          ok = false;
          break;
        }
        for (int f = 0; f < T.n_ff; ++f) {
          T.ffw[f] = L.ffw[f];
          T.ffb[f] = L.ffb[f];
          T.ffrows[f] = L.ffrows[f];
          T.ffcols[f] = L.ffcols[f];
          T.ffact[f] = L.ffact[f];
        }
        T.kcache = L.kcache;
        T.vcache = L.vcache;
        ok = cdml_tiny_layer_check(&T, D) == CDML_OK;
      }
      if (ok) {
        void *dev = nullptr;
        if (!tl.empty()) {
          check(cdml_malloc(&dev, tl.size() * sizeof(cdml_tiny_layer)), "cdml_malloc");
          allocs_.push_back(dev);
          check(cdml_memcpy_h2d_async(dev, tl.data(), tl.size() * sizeof(cdml_tiny_layer), stream_), "upload");
        }
        tiny_.embedding = emb_;
        tiny_.out_w = outproj_;
        tiny_.out_b = outbias_;
        tiny_.rope_cs = rope_cs_;
        tiny_.layers = static_cast<const cdml_tiny_layer *>(dev);
        tiny_.n_layers = (int)tl.size();
        tiny_.dim = D;
        tiny_.heads = cfg_.NumHeads;
        tiny_.vocab = cfg_.VocabSize;
        tiny_.max_seq = S;
        tiny_.eps = 1e-5f;
        tiny_ok_ = true;
      }
    }
    synchronize();
  } catch (...) {
    for (void *p : allocs_) cdml_free(p);
    cdml_stream_destroy(stream_);
    throw;
  }
}

DeviceLanguageModel::~DeviceLanguageModel() {
  cdml_stream_synchronize(stream_);
  for (auto &kv : graphs_) cdml_graph_destroy(kv.second);
  for (void *p : allocs_) cdml_free(p);
  cdml_stream_destroy(stream_);
}

void DeviceLanguageModel::synchronize() { check(cdml_stream_synchronize(stream_), "cdml_stream_synchronize"); }

// The blocks over x [batch * seqLen, D] in place (LanguageModel.cs:210-223 /
// TransformerBlock.cs:35-44), every sequence at positions 0..seqLen-1.  With
// fill_cache the post-RoPE K and V rows are also written to each layer's
// decode cache.
void DeviceLanguageModel::hidden_pass(float *x, int batch, int seqLen, bool fill_cache) {
  const int D = cfg_.EmbeddingDim, H = cfg_.NumHeads, hd = D / H, S = cfg_.MaxSequenceLength;
  const int rows = batch * seqLen;
  const float scale = 1.0f / std::sqrt((float)hd);
  for (auto &L : layers_) {
    // ProjectQKV + RoPE on Q and K (MultiHeadAttention.cs:108-110) in one launch
    check(cdml_project_qkv_rope(x, L.wq, L.bq, L.wk, L.bk, L.wv, L.bv, q_, k_, v_, rows, D, D, hd,
                                rope_cs_, S, 0, seqLen, stream_),
          "cdml_project_qkv_rope");
    if (fill_cache) {
      const size_t rowb = (size_t)seqLen * D * sizeof(float), pitch = (size_t)S * D * sizeof(float);
      check(cdml_memcpy2d_d2d_async(L.kcache, pitch, k_, rowb, rowb, batch, stream_), "cache fill");
      check(cdml_memcpy2d_d2d_async(L.vcache, pitch, v_, rowb, rowb, batch, stream_), "cache fill");
    }
    check(cdml_sdpa_fwd(q_, D, k_, D, v_, D, att_, D, batch, seqLen, seqLen, D, H, scale,
                        cfg_.UseDecoderOnly ? 1 : 0, nullptr, stream_),
          "cdml_sdpa_fwd");
    check(cdml_linear(att_, D, L.wo, L.bo, proj_, D, rows, D, D, CDML_ACT_NONE, stream_), "cdml_linear");
    check(cdml_residual_layernorm(x, proj_, L.ln1g, L.ln1b, h_, rows, D, 1e-5f, stream_), "layernorm");
    const float *in = h_;
    int width = D;
    float *bufs[2] = {ff_, ff2_};
    for (size_t l = 0; l < L.ffw.size(); ++l) {
      float *out = bufs[l & 1];
      check(cdml_linear(in, width, L.ffw[l], L.ffb[l], out, L.ffrows[l], rows, width, L.ffrows[l],
                        L.ffact[l], stream_),
            "cdml_linear");
      in = out;
      width = L.ffrows[l];
    }
    check(cdml_residual_layernorm(h_, in, L.ln2g, L.ln2b, x, rows, D, 1e-5f, stream_), "layernorm");
  }
}

void DeviceLanguageModel::layers_device(float *dev_x, int batch, int seqLen) {
  if (batch <= 0 || batch > cap_) throw ArgumentOutOfRangeException("batch");
  if (seqLen <= 0 || seqLen > cfg_.MaxSequenceLength) throw ArgumentOutOfRangeException("seqLen");
  hidden_pass(dev_x, batch, seqLen, false);
}

void DeviceLanguageModel::forward_device(const int *dev_ids, const float *dev_x, int batch,
                                         int seqLen, float *dev_out) {
  const int D = cfg_.EmbeddingDim, O = cfg_.EffectiveOutputDim();
  const int rows = batch * seqLen;
  if (cfg_.UsesDiscreteTokens)
    check(cdml_embed_tokens(dev_ids, rows, emb_, cfg_.VocabSize, D, x_, nullptr, stream_), "embed");
  else
    check(cdml_linear(dev_x, cfg_.InputFeatureDim, inproj_, inbias_, x_, D, rows, cfg_.InputFeatureDim,
                      D, CDML_ACT_NONE, stream_),
          "input projection");
  hidden_pass(x_, batch, seqLen, false);
  check(cdml_linear(x_, D, outproj_, outbias_, dev_out, O, rows, D, O, CDML_ACT_NONE, stream_),
        "output projection");
}

Matrix DeviceLanguageModel::Forward(const std::vector<int> &ids, int batch, int seqLen) {
  if (!cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Use ForwardContinuous for continuous input data types.");
  if (batch <= 0 || batch > cap_) throw ArgumentOutOfRangeException("batch");
  if (seqLen <= 0 || seqLen > cfg_.MaxSequenceLength) throw ArgumentOutOfRangeException("seqLen");
  if ((long long)ids.size() != (long long)batch * seqLen) throw ArgumentException("ids must hold batch * seqLen tokens.", "ids");
  for (size_t i = 0; i < ids.size(); ++i)
    if ((unsigned)ids[i] >= (unsigned)cfg_.VocabSize)
      throw ArgumentOutOfRangeException("ids", "Token id " + std::to_string(ids[i]) + " is outside the vocabulary.");
  const int O = cfg_.EffectiveOutputDim(), rows = batch * seqLen;
  check(cdml_memcpy_h2d_async(ids_, ids.data(), ids.size() * sizeof(int), stream_), "upload ids");
  forward_device(ids_, nullptr, batch, seqLen, logits_);
  Matrix out(rows, O);
  check(cdml_memcpy_d2h_async(out.ptr(), logits_, (size_t)rows * O * sizeof(float), stream_), "download");
  synchronize();
  return out;
}

Matrix DeviceLanguageModel::ForwardContinuous(MatView x, int batch, int seqLen) {
  if (cfg_.UsesDiscreteTokens) throw InvalidOperationException("Use Forward for discrete token data types.");
  if (x.null()) throw ArgumentNullException("x");
  if (batch <= 0 || batch > cap_) throw ArgumentOutOfRangeException("batch");
  if (seqLen <= 0 || seqLen > cfg_.MaxSequenceLength) throw ArgumentOutOfRangeException("seqLen");
  if (x.rows != batch * seqLen || x.cols != cfg_.InputFeatureDim)
    throw ArgumentException("x must be [batch * seqLen, InputFeatureDim].", "x");
  const int O = cfg_.EffectiveOutputDim(), rows = batch * seqLen;
  float *dx = ff_;  // the FFN buffer is free before the blocks run
  check(cdml_memcpy_h2d_async(dx, x.data, (size_t)rows * x.cols * sizeof(float), stream_), "upload x");
  forward_device(nullptr, dx, batch, seqLen, logits_);
  Matrix out(rows, O);
  check(cdml_memcpy_d2h_async(out.ptr(), logits_, (size_t)rows * O * sizeof(float), stream_), "download");
  synchronize();
  return out;
}

// One token per sequence at absolute position pos (LanguageModel.cs:305-430):
// dev_tok [batch] device token ids; leaves the hidden rows in x [batch, D].
void DeviceLanguageModel::decode_step(const int *dev_tok, int batch, int pos, float *x) {
  const int D = cfg_.EmbeddingDim, H = cfg_.NumHeads, hd = D / H, S = cfg_.MaxSequenceLength;
  const float scale = 1.0f / std::sqrt((float)hd);
  check(cdml_embed_tokens(dev_tok, batch, emb_, cfg_.VocabSize, D, x, nullptr, stream_), "embed");
  check(cdml_fill_i32_async(pos_, batch, pos, stream_), "positions");
  check(cdml_fill_i32_async(kvlen_, batch, pos + 1, stream_), "kv lengths");
  for (auto &L : layers_) {
    // every row at position pos (seg_len 1)
    check(cdml_project_qkv_rope(x, L.wq, L.bq, L.wk, L.bk, L.wv, L.bv, q_, k_, v_, batch, D, D, hd,
                                rope_cs_, S, pos, 1, stream_),
          "cdml_project_qkv_rope");
    check(cdml_kv_cache_append(k_, v_, L.kcache, L.vcache, pos_, batch, S, D, stream_), "kv append");
    check(cdml_decode_attn(q_, L.kcache, L.vcache, kvlen_, att_, batch, S, D, H, scale, ws_, ws_bytes_,
                           stream_),
          "cdml_decode_attn");
    check(cdml_linear(att_, D, L.wo, L.bo, proj_, D, batch, D, D, CDML_ACT_NONE, stream_), "cdml_linear");
    check(cdml_residual_layernorm(x, proj_, L.ln1g, L.ln1b, h_, batch, D, 1e-5f, stream_), "layernorm");
    const float *in = h_;
    int width = D;
    float *bufs[2] = {ff_, ff2_};
    for (size_t l = 0; l < L.ffw.size(); ++l) {
      float *out = bufs[l & 1];
      check(cdml_linear(in, width, L.ffw[l], L.ffb[l], out, L.ffrows[l], batch, width, L.ffrows[l],
                        L.ffact[l], stream_),
            "cdml_linear");
      in = out;
      width = L.ffrows[l];
    }
    check(cdml_residual_layernorm(h_, in, L.ln2g, L.ln2b, x, batch, D, 1e-5f, stream_), "layernorm");
  }
}

// The device work of one greedy generation after the prompt ids are in
// ids_: the prompt prefilled in one pass, then n - 1 decode steps; token s of
// every sequence lands in gen_[s * batch + b].  Only enqueue calls, so the
// sequence can be recorded as a graph.
void DeviceLanguageModel::generate_device(int batch, int promptLen, int n) {
  const int D = cfg_.EmbeddingDim, V = cfg_.VocabSize;
  check(cdml_embed_tokens(ids_, batch * promptLen, emb_, V, D, x_, nullptr, stream_), "embed");
  hidden_pass(x_, batch, promptLen, true);
  // logits of each sequence's last prompt position: rows (P-1), stride P*D
  check(cdml_linear(x_ + (size_t)(promptLen - 1) * D, promptLen * D, outproj_, outbias_, logits_, V,
                    batch, D, V, CDML_ACT_NONE, stream_),
        "output projection");
  check(cdml_argmax_rows(logits_, batch, V, V, gen_, 1, stream_), "argmax");
  if (use_fused_decode && tiny_ok_ && n > 1) {  // every later step in one launch
    check(cdml_tiny_decode(&tiny_, gen_, batch, promptLen, n - 1, stream_), "cdml_tiny_decode");
    return;
  }
  for (int s = 1; s < n; ++s) {
    decode_step(gen_ + (size_t)(s - 1) * batch, batch, promptLen + s - 1, x_);
    check(cdml_linear(x_, D, outproj_, outbias_, logits_, V, batch, D, V, CDML_ACT_NONE, stream_),
          "output projection");
    check(cdml_argmax_rows(logits_, batch, V, V, gen_ + (size_t)s * batch, 1, stream_), "argmax");
  }
}

// LanguageModel.Generate (:482-537) for a batch of equal-length prompts with
// greedy selection: the prompt is prefilled in one pass (instead of one token
// at a time), then every new token runs one decode step per sequence; token
// choice (cdml_argmax_rows) and the KV caches stay on the device.
std::vector<int> DeviceLanguageModel::GenerateGreedy(const std::vector<int> &prompts, int batch,
                                                     int promptLen, int maxNewTokens, int *outLen) {
  if (!cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("Generate is only supported for discrete token data types.");
  if (batch <= 0 || batch > cap_) throw ArgumentOutOfRangeException("batch");
  if (promptLen <= 0) throw ArgumentException("Token sequence must contain at least one token.", "tokenIds");
  if (promptLen > cfg_.MaxSequenceLength)
    throw ArgumentException("Token sequence length exceeds MaxSequenceLength.", "tokenIds");
  if ((long long)prompts.size() != (long long)batch * promptLen)
    throw ArgumentException("prompts must hold batch * promptLen tokens.", "prompts");
  for (int t : prompts)
    if ((unsigned)t >= (unsigned)cfg_.VocabSize) throw ArgumentOutOfRangeException("tokenIds");
  if (maxNewTokens < 0) throw ArgumentOutOfRangeException("maxNewTokens", "maxNewTokens must be non-negative.");
  const int S = cfg_.MaxSequenceLength, D = cfg_.EmbeddingDim, V = cfg_.VocabSize;
  const int n = (promptLen >= S || maxNewTokens == 0) ? 0 : std::min(maxNewTokens, S - promptLen);
  const int total = promptLen + n;
  std::vector<int> out((size_t)batch * total);
  for (int b = 0; b < batch; ++b)
    std::copy(prompts.begin() + (size_t)b * promptLen, prompts.begin() + (size_t)(b + 1) * promptLen,
              out.begin() + (size_t)b * total);
  if (outLen) *outLen = total;
  if (n == 0) return out;

  check(cdml_memcpy_h2d_async(ids_, prompts.data(), prompts.size() * sizeof(int), stream_), "upload ids");
  if (cfg_.UseDecoderOnly) {
    if (use_graphs) {
      // the recording holds the decode path chosen at capture time, so the
      // path's switch is part of the key
      const bool fused = use_fused_decode && tiny_ok_ && n > 1;
      const auto key = std::make_tuple(batch, promptLen, n, fused);
      auto it = graphs_.find(key);
      if (it == graphs_.end()) {
        if (graphs_.size() >= 16) {  // a bounded cache: drop every recording
          synchronize();
          for (auto &kv : graphs_) cdml_graph_destroy(kv.second);
          graphs_.clear();
        }
        check(cdml_graph_capture_begin(stream_), "cdml_graph_capture_begin");
        cdml_graph g = nullptr;
        try {
          generate_device(batch, promptLen, n);
        } catch (...) {
          cdml_graph_capture_end(stream_, &g);  // discards the partial recording
          cdml_graph_destroy(g);
          throw;
        }
        check(cdml_graph_capture_end(stream_, &g), "cdml_graph_capture_end");
        it = graphs_.emplace(key, g).first;
      }
      check(cdml_graph_launch(it->second, stream_), "cdml_graph_launch");
    } else {
      generate_device(batch, promptLen, n);
    }
    std::vector<int> gen((size_t)n * batch);
    check(cdml_memcpy_d2h_async(gen.data(), gen_, gen.size() * sizeof(int), stream_), "download");
    synchronize();
    for (int s = 0; s < n; ++s)
      for (int b = 0; b < batch; ++b) out[(size_t)b * total + promptLen + s] = gen[(size_t)s * batch + b];
    return out;
  }
  // Encoder-style models recompute the whole prefix per token (:500-512).
  std::vector<int> cur(prompts);
  for (int s = 0; s < n; ++s) {
    const int len = promptLen + s;
    check(cdml_memcpy_h2d_async(ids_, cur.data(), cur.size() * sizeof(int), stream_), "upload ids");
    check(cdml_embed_tokens(ids_, batch * len, emb_, V, D, x_, nullptr, stream_), "embed");
    hidden_pass(x_, batch, len, false);
    check(cdml_linear(x_ + (size_t)(len - 1) * D, len * D, outproj_, outbias_, logits_, V, batch, D, V,
                      CDML_ACT_NONE, stream_),
          "output projection");
    check(cdml_argmax_rows(logits_, batch, V, V, gen_, 1, stream_), "argmax");
    std::vector<int> next(batch);
    check(cdml_memcpy_d2h_async(next.data(), gen_, batch * sizeof(int), stream_), "download");
    synchronize();
    std::vector<int> grown((size_t)batch * (len + 1));
    for (int b = 0; b < batch; ++b) {
      std::copy(cur.begin() + (size_t)b * len, cur.begin() + (size_t)(b + 1) * len,
                grown.begin() + (size_t)b * (len + 1));
      grown[(size_t)b * (len + 1) + len] = next[b];
      out[(size_t)b * total + len] = next[b];
    }
    cur.swap(grown);
  }
  return out;
}

}  // namespace cdml_host
