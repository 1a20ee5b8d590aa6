// TransformerTrainer (Transformers/MultiTypeTransformer/TransformerTrainer.cs)
// restated on HipAccelerationManager for token and continuous-input models:
// the reference's call sequence, one manager call per `_accel.X(...)`, with
// the model's host arrays updated in place.  Line references are to that file
// unless another is named.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "cdml_host.h"

namespace cdml_host {

namespace {

bool is_finite(float v) { return !std::isnan(v) && !std::isinf(v); }

// MatrixAllFinite (:1511-1523), the trainer's own host check.
bool all_finite(const Matrix &m) {
  for (float v : m.data)
    if (!is_finite(v)) return false;
  return true;
}

MatRef ref(Matrix &m) { return MatRef(m.ptr(), m.rows, m.cols); }
VecRef ref(std::vector<float> &v) { return VecRef(v.data(), (int)v.size()); }

// MatrixAllFinite over a view
bool all_finite(MatView m) {
  for (size_t i = 0, n = (size_t)m.rows * m.cols; i < n; ++i)
    if (!is_finite(m.data[i])) return false;
  return true;
}

// ShuffleInPlace (:1417-1430): Fisher-Yates from the last element, j drawn
// in [0, i]; the draws come from SplitMix64 (the reference's System.Random
// stream is not reproduced).
struct SplitMix64 {
  uint64_t state;
  uint64_t next() {
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
};
template <class T>
void shuffle_in_place(std::vector<T> &data, SplitMix64 &rng) {
  for (size_t i = data.size(); i > 1; --i) std::swap(data[i - 1], data[rng.next() % i]);
}

constexpr int kTimeSeriesRegression = 1;  // TransformerDataType.TimeSeriesRegression

}  // namespace

TransformerTrainer::TransformerTrainer(LanguageModel &model, const TrainingConfig &config)
    : model_(model), cfg_(model.config()), tc_(new TrainingConfig(config)), accel_(model.AccelerationManager()) {
  const int D = cfg_.EmbeddingDim, L = cfg_.NumLayers, V = cfg_.EffectiveOutputDim();
  // TransformerGradients(config) (TransformerGradients.cs:28-60)
  if (cfg_.UsesDiscreteTokens) {
    grads_.TokenEmbeddingGrad = Matrix(cfg_.VocabSize, D);
    grads_.marked.assign(cfg_.VocabSize, 0);
  } else {
    grads_.InputProjectionGrad = Matrix(D, cfg_.InputFeatureDim);
    grads_.InputProjectionBiasGrad.assign(D, 0.f);
  }
  grads_.OutputProjectionGrad = Matrix(V, D);
  grads_.OutputBiasGrad.assign(V, 0.f);
  for (int i = 0; i < L; ++i) {
    AttentionGradients a;
    a.WQ_Grad = Matrix(D, D);
    a.WK_Grad = Matrix(D, D);
    a.WV_Grad = Matrix(D, D);
    a.WO_Grad = Matrix(D, D);
    a.BiasQ_Grad.assign(D, 0.f);
    a.BiasK_Grad.assign(D, 0.f);
    a.BiasV_Grad.assign(D, 0.f);
    a.BiasO_Grad.assign(D, 0.f);
    grads_.AttentionGrads.push_back(std::move(a));
    grads_.LN1Grads.push_back(LayerNormGradients{std::vector<float>(D, 0.f), std::vector<float>(D, 0.f)});
    grads_.LN2Grads.push_back(LayerNormGradients{std::vector<float>(D, 0.f), std::vector<float>(D, 0.f)});
    // FeedForwardNetwork.CreateGradientStorage (NeuralNetwork.cs:1021-1035)
    const FeedForwardNetwork &f = model_.Blocks[i].FeedForward;
    std::vector<Matrix> wg;
    std::vector<std::vector<float>> bg;
    for (size_t l = 0; l < f.weights.size(); ++l) {
      wg.emplace_back(f.weights[l].rows, f.weights[l].cols);
      bg.emplace_back(f.weights[l].rows, 0.f);
    }
    ffnWeightGrads_.push_back(std::move(wg));
    ffnBiasGrads_.push_back(std::move(bg));
  }
}

TransformerTrainer::~TransformerTrainer() = default;

// ---- Train / TrainBatchDiscrete ----------------------------------------------
float TransformerTrainer::Train(const std::vector<std::vector<int>> &sequences, uint64_t seed,
                                const std::vector<std::vector<int>> *validationSequences) {
  if (!cfg_.UsesDiscreteTokens) throw InvalidOperationException("Use TrainContinuous() for continuous data types.");
  if (tc_->BatchSize <= 0) throw ArgumentOutOfRangeException("BatchSize", "BatchSize must be positive.");
  if (tc_->Epochs < 0) throw ArgumentOutOfRangeException("Epochs", "Epochs must be non-negative.");
  std::vector<std::vector<int>> valid;
  for (const auto &s : sequences)
    if (s.size() >= 2) valid.push_back(s);
  if (valid.empty())
    throw ArgumentException("No valid sequences to train on. All sequences must contain at least 2 tokens.",
                            "sequences");
  float lr = tc_->LearningRate, epochAvg = 0.f;
  SplitMix64 rng{seed};
  val_losses_.clear();
  for (int epoch = 0; epoch < tc_->Epochs; ++epoch) {
    std::vector<std::vector<int>> order = valid;  // ShuffleArray: a shuffled copy
    shuffle_in_place(order, rng);
    float epochLoss = 0.f;
    int numBatches = 0;
    for (size_t i = 0; i < order.size(); i += tc_->BatchSize) {
      std::vector<std::vector<int>> b(order.begin() + i,
                                      order.begin() + std::min(order.size(), i + (size_t)tc_->BatchSize));
      epochLoss += TrainBatch(b, lr);
      ++numBatches;
      // :92-104
      if (validationSequences && tc_->ValidationInterval > 0 && numBatches % tc_->ValidationInterval == 0)
        val_losses_.push_back(Validate(*validationSequences));
    }
    epochAvg = numBatches > 0 ? epochLoss / numBatches : 0.f;
    if (tc_->UseLearningRateDecay) lr *= tc_->LearningRateDecay;
  }
  return epochAvg;
}

// ---- TrainContinuous / TrainBatchContinuous (:130-207, :329-512) ---------------
float TransformerTrainer::TrainContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> *regressionTargets,
                                          const std::vector<std::vector<int>> *classTargets, uint64_t seed) {
  if (cfg_.UsesDiscreteTokens) throw InvalidOperationException("Use Train(int[][]) for discrete token data types.");
  if (tc_->BatchSize <= 0) throw ArgumentOutOfRangeException("BatchSize", "BatchSize must be positive.");
  if (tc_->Epochs < 0) throw ArgumentOutOfRangeException("Epochs", "Epochs must be non-negative.");
  if (cfg_.DataType == kTimeSeriesRegression) {
    if (!regressionTargets)
      throw ArgumentException("regressionTargets is required for TimeSeriesRegression.", "regressionTargets");
    if (regressionTargets->size() != inputs.size())
      throw ArgumentException("regressionTargets length must match inputs length.", "regressionTargets");
  } else {  // TimeSeriesClassification (:150-156)
    if (!classTargets)
      throw ArgumentException("classTargets is required for TimeSeriesClassification.", "classTargets");
    if (classTargets->size() != inputs.size())
      throw ArgumentException("classTargets length must match inputs length.", "classTargets");
  }
  std::vector<int> validIndices;
  for (int i = 0; i < (int)inputs.size(); ++i) {
    if (inputs[i].rows < 2) continue;
    if (inputs[i].cols != cfg_.InputFeatureDim)
      throw ArgumentException("Input sequence " + std::to_string(i) + " has feature dimension " +
                                  std::to_string(inputs[i].cols) + ", expected " +
                                  std::to_string(cfg_.InputFeatureDim) + ".",
                              "inputs");
    validIndices.push_back(i);
  }
  if (validIndices.empty())
    throw ArgumentException("No valid sequences. All must have at least 2 timesteps.", "inputs");
  float lr = tc_->LearningRate, epochAvg = 0.f;
  SplitMix64 rng{seed};
  for (int epoch = 0; epoch < tc_->Epochs; ++epoch) {
    std::vector<int> shuffled = validIndices;
    shuffle_in_place(shuffled, rng);
    float epochLoss = 0.f;
    int numBatches = 0;
    for (int i = 0; i < (int)shuffled.size(); i += tc_->BatchSize) {
      const int batchSize = std::min(tc_->BatchSize, (int)shuffled.size() - i);
      if (batchSize == 0) continue;
      epochLoss += TrainBatchContinuousRange(shuffled, i, batchSize, inputs, regressionTargets, classTargets, lr);
      ++numBatches;
    }
    epochAvg = numBatches > 0 ? epochLoss / numBatches : 0.f;
    if (tc_->UseLearningRateDecay) lr *= tc_->LearningRateDecay;
  }
  return epochAvg;
}

float TransformerTrainer::TrainBatchContinuous(const std::vector<Matrix> &inputs,
                                               const std::vector<Matrix> *regressionTargets,
                                               const std::vector<std::vector<int>> *classTargets,
                                               float learningRate) {
  if (cfg_.UsesDiscreteTokens)
    throw InvalidOperationException("TrainBatchContinuous needs a continuous-input model.");
  std::vector<int> indices(inputs.size());
  for (size_t i = 0; i < indices.size(); ++i) indices[i] = (int)i;
  return TrainBatchContinuousRange(indices, 0, (int)indices.size(), inputs, regressionTargets, classTargets,
                                   learningRate);
}

// RegressionTargetIsValid / ClassTargetIsValid (:1480-1502)
bool TransformerTrainer::RegressionTargetIsValid(const std::vector<Matrix> *targets, int idx, int seqLen) const {
  if (!targets || idx < 0 || idx >= (int)targets->size()) return false;
  const Matrix &t = (*targets)[idx];
  return t.rows > 0 && t.rows >= seqLen && t.cols == cfg_.OutputDim && all_finite(MatView(t));
}

bool TransformerTrainer::ClassTargetIsValid(const std::vector<std::vector<int>> *targets, int idx, int seqLen) const {
  if (!targets || idx < 0 || idx >= (int)targets->size()) return false;
  const std::vector<int> &t = (*targets)[idx];
  if (t.empty() || (int)t.size() < seqLen) return false;
  for (int i = 1; i < seqLen; ++i)
    if ((unsigned)t[i] >= (unsigned)cfg_.OutputDim) return false;
  return true;
}

float TransformerTrainer::TrainBatchContinuousRange(const std::vector<int> &batchIndices, int start, int count,
                                                    const std::vector<Matrix> &allInputs,
                                                    const std::vector<Matrix> *allRegTargets,
                                                    const std::vector<std::vector<int>> *allClassTargets,
                                                    float learningRate) {
  if (start < 0 || count < 0 || (long long)start + count > (long long)batchIndices.size())
    throw ArgumentOutOfRangeException("start");
  ZeroAllGradients();
  float totalLoss = 0.f;
  int validCount = 0;
  const bool regression = cfg_.DataType == kTimeSeriesRegression;
  // buckets in order of first appearance (:351-386)
  std::vector<std::pair<int, std::vector<int>>> buckets;
  for (int batchOffset = 0; batchOffset < count; ++batchOffset) {
    const int idx = batchIndices[start + batchOffset];
    if ((unsigned)idx >= (unsigned)allInputs.size()) continue;
    const Matrix &inputSeq = allInputs[idx];
    const int seqLen = inputSeq.rows;
    if (seqLen < 2 || inputSeq.cols != cfg_.InputFeatureDim) continue;
    if (!all_finite(MatView(inputSeq))) continue;
    if (regression ? !RegressionTargetIsValid(allRegTargets, idx, seqLen)
                   : !ClassTargetIsValid(allClassTargets, idx, seqLen))
      continue;
    const int inputLen = seqLen - 1;
    auto it = std::find_if(buckets.begin(), buckets.end(), [&](const auto &b) { return b.first == inputLen; });
    if (it == buckets.end()) {
      buckets.emplace_back(inputLen, std::vector<int>());
      it = buckets.end() - 1;
    }
    it->second.push_back(idx);
  }
  for (auto &bucket : buckets) {
    const int inputLen = bucket.first;
    const std::vector<int> &sourceIndices = bucket.second;
    if (sourceIndices.empty()) continue;
    const int n = (int)sourceIndices.size();
    try {
      ForwardCache cache;
      Matrix output = n == 1 ? ForwardWithCacheContinuous(allInputs[sourceIndices[0]], 0, inputLen, cache)
                             : ForwardWithCacheContinuousBatch(sourceIndices, allInputs, inputLen, cache);
      const int effectiveLen = std::min(output.rows, n * inputLen);
      if (effectiveLen <= 0) continue;
      std::pair<float, Matrix> r;
      if (regression) {
        if (n == 1) {
          r = accel_->MSELossAndGradient(output, (*allRegTargets)[sourceIndices[0]], 1,
                                         std::min(output.rows, inputLen));
        } else {
          // BuildContinuousRegressionFlatTargets (:690-708)
          const int outputDim = cfg_.EffectiveOutputDim();
          Matrix targets(n * inputLen, outputDim);
          for (int b = 0; b < n; ++b) {
            const Matrix &src = (*allRegTargets)[sourceIndices[b]];
            for (int t = 0; t < inputLen; ++t)
              for (int o = 0; o < outputDim; ++o) targets.at(b * inputLen + t, o) = src.at(t + 1, o);
          }
          r = accel_->MSELossAndGradient(output, targets, 0, effectiveLen);
        }
      } else {
        if (n == 1) {
          r = accel_->CrossEntropyLossAndGradient(output, (*allClassTargets)[sourceIndices[0]], 1,
                                                  std::min(output.rows, inputLen));
        } else {
          // BuildContinuousClassFlatTargets (:676-688)
          std::vector<int> targets((size_t)n * inputLen);
          for (int b = 0; b < n; ++b)
            for (int t = 0; t < inputLen; ++t)
              targets[(size_t)b * inputLen + t] = (*allClassTargets)[sourceIndices[b]][t + 1];
          r = accel_->CrossEntropyLossAndGradient(output, targets, 0, effectiveLen);
        }
      }
      if (!is_finite(r.first) || !all_finite(r.second)) continue;
      if (n > 1)  // ScaleMatrixLocal (:710-721)
        for (float &x : r.second.data) x *= (float)n;
      BackpropFromOutput(r.second, cache);
      totalLoss += r.first * (float)n;
      validCount += n;
    } catch (const std::exception &) {  // :470-478
      ZeroAllGradients();
      totalLoss = 0.f;
      validCount = 0;
    }
  }
  if (validCount == 0) return 0.f;
  ScaleGradients(1.0f / validCount);
  const float gradNorm = ComputeGradientNorm();
  last_norm_ = gradNorm;
  if (!is_finite(gradNorm)) {
    ZeroAllGradients();
    return totalLoss / validCount;
  }
  if (tc_->UseGradientClipping) ClipGradients(tc_->GradientClipThreshold, gradNorm);
  UpdateParameters(learningRate);
  return totalLoss / validCount;
}

// ---- Validate / ValidateContinuous (:1142-1267) --------------------------------
float TransformerTrainer::Validate(const std::vector<std::vector<int>> &validationSequences) {
  float totalLoss = 0.f;
  int totalTokens = 0;
  for (const std::vector<int> &sequence : validationSequences) {
    if (sequence.size() < 2) continue;
    bool ok = true;  // TokensAreValid (:1467-1478)
    for (int t : sequence)
      if ((unsigned)t >= (unsigned)cfg_.VocabSize) ok = false;
    if (!ok) continue;
    const int inputLen = (int)sequence.size() - 1;
    Matrix logits = model_.ForwardTokenSlice(sequence, 0, inputLen);
    const int effectiveLen = std::min(logits.rows, inputLen);
    if (effectiveLen <= 0) continue;
    auto r = accel_->CrossEntropyLossAndGradient(logits, sequence, 1, effectiveLen);
    if (!is_finite(r.first)) continue;
    totalLoss += r.first * effectiveLen;
    totalTokens += effectiveLen;
  }
  return totalTokens > 0 ? totalLoss / totalTokens : 0.0f;
}

float TransformerTrainer::ValidateContinuous(const std::vector<Matrix> &inputs,
                                             const std::vector<Matrix> *regressionTargets,
                                             const std::vector<std::vector<int>> *classTargets) {
  float totalLoss = 0.f;
  int totalItems = 0;
  const bool regression = cfg_.DataType == kTimeSeriesRegression;
  for (int idx = 0; idx < (int)inputs.size(); ++idx) {
    const Matrix &inputSeq = inputs[idx];
    const int seqLen = inputSeq.rows;
    if (seqLen < 2) continue;  // a null window and a short one alike
    const int inputLen = seqLen - 1;
    Matrix output = model_.ForwardContinuousSlice(inputSeq, 0, inputLen);
    int effectiveLen = output.rows;
    // regressionTargets[idx] / classTargets[idx] past the array's end throw
    // IndexOutOfRangeException in the reference
    if (regression) {
      if (!regressionTargets) continue;
      if (idx >= (int)regressionTargets->size()) throw ArgumentOutOfRangeException("regressionTargets");
      const Matrix &t = (*regressionTargets)[idx];
      if (t.rows == 0) continue;
      effectiveLen = std::min(effectiveLen, inputLen);
      if (effectiveLen <= 0) continue;
      auto r = accel_->MSELossAndGradient(output, t, 1, effectiveLen);
      if (!is_finite(r.first)) continue;
      totalLoss += r.first * effectiveLen;
      totalItems += effectiveLen;
    } else {
      if (!classTargets) continue;
      if (idx >= (int)classTargets->size()) throw ArgumentOutOfRangeException("classTargets");
      const std::vector<int> &t = (*classTargets)[idx];
      if (t.empty()) continue;
      effectiveLen = std::min(effectiveLen, inputLen);
      if (effectiveLen <= 0) continue;
      auto r = accel_->CrossEntropyLossAndGradient(output, t, 1, effectiveLen);
      if (!is_finite(r.first)) continue;
      totalLoss += r.first * effectiveLen;
      totalItems += effectiveLen;
    }
  }
  return totalItems > 0 ? totalLoss / totalItems : 0.0f;
}

float TransformerTrainer::TrainBatch(const std::vector<std::vector<int>> &batch, float learningRate) {
  if (!cfg_.UsesDiscreteTokens) throw InvalidOperationException("TrainBatchDiscrete needs a token model.");
  ZeroAllGradients();
  float totalLoss = 0.f;
  int validCount = 0;
  // length buckets in order of first appearance (a Dictionary without
  // removals enumerates in insertion order), :229-248
  std::vector<std::pair<int, std::vector<int>>> buckets;
  for (int i = 0; i < (int)batch.size(); ++i) {
    const std::vector<int> &seq = batch[i];
    if (seq.size() < 2) continue;
    bool ok = true;  // TokensAreValid (:1467-1478)
    for (int t : seq)
      if ((unsigned)t >= (unsigned)cfg_.VocabSize) ok = false;
    if (!ok) continue;
    const int inputLen = (int)seq.size() - 1;
    auto it = std::find_if(buckets.begin(), buckets.end(), [&](const auto &b) { return b.first == inputLen; });
    if (it == buckets.end()) {
      buckets.emplace_back(inputLen, std::vector<int>());
      it = buckets.end() - 1;
    }
    it->second.push_back(i);
  }
  for (auto &bucket : buckets) {
    const int inputLen = bucket.first;
    const std::vector<int> &offsets = bucket.second;
    if (offsets.empty()) continue;
    try {
      ForwardCache cache;
      if (offsets.size() == 1) {
        const std::vector<int> &sequence = batch[offsets[0]];
        Matrix logits = ForwardWithCacheDiscrete(sequence, 0, inputLen, cache);
        const int effectiveSingle = std::min(logits.rows, inputLen);
        if (effectiveSingle <= 0) continue;
        auto r = accel_->CrossEntropyLossAndGradient(logits, sequence, 1, effectiveSingle);
        if (!is_finite(r.first) || !all_finite(r.second)) continue;
        BackpropFromOutput(r.second, cache);
        totalLoss += r.first;
        validCount++;
      } else {
        Matrix logits = ForwardWithCacheDiscreteBatch(batch, offsets, inputLen, cache);
        // BuildDiscreteFlatTargets (:660-674)
        std::vector<int> targets((size_t)offsets.size() * inputLen);
        for (size_t b = 0; b < offsets.size(); ++b)
          for (int t = 0; t < inputLen; ++t) targets[b * inputLen + t] = batch[offsets[b]][t + 1];
        const int effectiveLen = std::min(logits.rows, (int)targets.size());
        if (effectiveLen <= 0) continue;
        auto r = accel_->CrossEntropyLossAndGradient(logits, targets, 0, effectiveLen);
        if (!is_finite(r.first) || !all_finite(r.second)) continue;
        // ScaleMatrixLocal (:710-721): the bucket's per-sample average gradients
        const float count = (float)offsets.size();
        for (float &x : r.second.data) x *= count;
        BackpropFromOutput(r.second, cache);
        totalLoss += r.first * (float)offsets.size();
        validCount += (int)offsets.size();
      }
    } catch (const std::exception &) {  // :293-302: a failed bucket voids the batch so far
      ZeroAllGradients();
      totalLoss = 0.f;
      validCount = 0;
    }
  }
  if (validCount == 0) return 0.f;
  ScaleGradients(1.0f / validCount);
  const float gradNorm = ComputeGradientNorm();
  last_norm_ = gradNorm;
  if (!is_finite(gradNorm)) {
    ZeroAllGradients();
    return totalLoss / validCount;
  }
  if (tc_->UseGradientClipping) ClipGradients(tc_->GradientClipThreshold, gradNorm);
  UpdateParameters(learningRate);
  return totalLoss / validCount;
}

// ---- forward with cache (:487-622) ---------------------------------------------
Matrix TransformerTrainer::ForwardWithCacheDiscrete(const std::vector<int> &tokenIds, int tokenStart, int tokenCount,
                                                    ForwardCache &cache) {
  if (tokenStart < 0 || tokenCount < 0 || (long long)tokenStart + tokenCount > (long long)tokenIds.size())
    throw ArgumentOutOfRangeException("tokenStart");
  auto embedded = std::make_shared<Matrix>(
      accel_->EmbedTokenIds(tokenIds, tokenStart, tokenCount, model_.TokenEmbedding, cfg_.EmbeddingDim));
  cache.EmbeddedInput = embedded;
  cache.TokenIds = tokenIds;
  cache.TokenStart = tokenStart;
  cache.TokenCount = tokenCount;
  return ForwardFromEmbeddingWithCache(embedded, tokenCount, cache);
}

Matrix TransformerTrainer::ForwardWithCacheDiscreteBatch(const std::vector<std::vector<int>> &sequences,
                                                         const std::vector<int> &offsets, int inputLen,
                                                         ForwardCache &cache) {
  if (inputLen <= 0) throw ArgumentOutOfRangeException("inputLen");
  const int batchSize = (int)offsets.size(), totalRows = batchSize * inputLen;
  std::vector<int> flat((size_t)totalRows);
  for (int b = 0; b < batchSize; ++b)
    for (int t = 0; t < inputLen; ++t) flat[(size_t)b * inputLen + t] = sequences[offsets[b]][t];
  auto embedded = std::make_shared<Matrix>(accel_->EmbedTokenIds(flat, model_.TokenEmbedding, cfg_.EmbeddingDim));
  cache.EmbeddedInput = embedded;
  cache.TokenIds = flat;
  cache.TokenStart = 0;
  cache.TokenCount = totalRows;
  return ForwardFromEmbeddingWithCache(embedded, totalRows, cache, inputLen, batchSize);
}

// :436-457
Matrix TransformerTrainer::ForwardWithCacheContinuous(MatView inputSequence, int rowStart, int rowCount,
                                                      ForwardCache &cache) {
  if (inputSequence.null()) throw ArgumentNullException("inputSequence");
  if (rowStart < 0 || rowCount < 0 || (long long)rowStart + rowCount > inputSequence.rows)
    throw ArgumentOutOfRangeException("rowStart");
  auto embedded = std::make_shared<Matrix>(accel_->BatchDotProductAddBias(
      model_.InputProjection, inputSequence, rowStart, rowCount, model_.InputProjectionBias));
  cache.EmbeddedInput = embedded;
  cache.TokenIds.clear();
  cache.TokenStart = 0;
  cache.TokenCount = 0;
  cache.ContinuousInput = inputSequence;
  cache.ContinuousInputRowStart = rowStart;
  cache.ContinuousInputRowCount = rowCount;
  return ForwardFromEmbeddingWithCache(embedded, rowCount, cache);
}

// :624-658
Matrix TransformerTrainer::ForwardWithCacheContinuousBatch(const std::vector<int> &sourceIndices,
                                                           const std::vector<Matrix> &allInputs, int inputLen,
                                                           ForwardCache &cache) {
  if (inputLen <= 0) throw ArgumentOutOfRangeException("inputLen");
  const int count = (int)sourceIndices.size(), totalRows = count * inputLen, F = cfg_.InputFeatureDim;
  auto flatInput = std::make_shared<Matrix>(totalRows, F);
  for (int b = 0; b < count; ++b) {
    const Matrix &source = allInputs[sourceIndices[b]];
    for (int t = 0; t < inputLen; ++t)
      for (int f = 0; f < F; ++f) flatInput->at(b * inputLen + t, f) = source.at(t, f);
  }
  auto embedded = std::make_shared<Matrix>(
      accel_->BatchDotProductAddBias(model_.InputProjection, *flatInput, model_.InputProjectionBias));
  cache.EmbeddedInput = embedded;
  cache.TokenIds.clear();
  cache.TokenStart = 0;
  cache.TokenCount = 0;
  cache.ContinuousOwned = flatInput;
  cache.ContinuousInput = *flatInput;
  cache.ContinuousInputRowStart = 0;
  cache.ContinuousInputRowCount = totalRows;
  return ForwardFromEmbeddingWithCache(embedded, totalRows, cache, inputLen, count);
}

Matrix TransformerTrainer::ForwardFromEmbeddingWithCache(MatPtr embedded, int seqLen, ForwardCache &cache,
                                                         int segmentLength, int segmentCount) {
  const bool selfCausal = cfg_.UseDecoderOnly;
  const int L = cfg_.NumLayers;
  cache.AttentionCaches.assign(L, AttentionCache{});
  cache.LN1Caches.assign(L, LayerNormCache{});
  cache.LN2Caches.assign(L, LayerNormCache{});
  MatPtr x = embedded;
  for (int layer = 0; layer < L; ++layer) {
    cache.LayerInputs.push_back(x);
    TransformerBlock &block = model_.Blocks[layer];
    AttentionCache &attnCache = cache.AttentionCaches[layer];
    attnCache.Input = x;
    MatPtr attnOutput = segmentCount > 1 ? SegmentedAttentionForwardWithCache(block.Attention, x, segmentLength,
                                                                              segmentCount, selfCausal, attnCache)
                                         : AttentionForwardWithCache(block.Attention, x, selfCausal, attnCache);
    auto ln1 = accel_->ResidualLayerNormForward(*x, *attnOutput, block.LN1Gamma, block.LN1Beta);
    LayerNormCache &c1 = cache.LN1Caches[layer];
    auto normed1 = std::make_shared<Matrix>(std::move(std::get<0>(ln1)));
    c1.Mean = std::move(std::get<1>(ln1));
    c1.Variance = std::move(std::get<2>(ln1));
    c1.Normalized = std::make_shared<Matrix>(std::move(std::get<3>(ln1)));
    c1.Input = std::make_shared<Matrix>(std::move(std::get<4>(ln1)));
    auto ffOutput = std::make_shared<Matrix>(
        accel_->FFNForwardBatch(*normed1, seqLen, cfg_.EmbeddingDim, block.FeedForward));
    cache.FFNInputs.push_back(normed1);
    cache.FFNOutputs.push_back(ffOutput);
    auto ln2 = accel_->ResidualLayerNormForward(*normed1, *ffOutput, block.LN2Gamma, block.LN2Beta);
    LayerNormCache &c2 = cache.LN2Caches[layer];
    auto normed2 = std::make_shared<Matrix>(std::move(std::get<0>(ln2)));
    c2.Mean = std::move(std::get<1>(ln2));
    c2.Variance = std::move(std::get<2>(ln2));
    c2.Normalized = std::make_shared<Matrix>(std::move(std::get<3>(ln2)));
    c2.Input = std::make_shared<Matrix>(std::move(std::get<4>(ln2)));
    x = normed2;
  }
  cache.FinalHiddenStates = x;
  // ProjectToOutput (:1396-1399)
  return accel_->ProjectOutputBatch(*x, model_.OutputProjection, model_.OutputBias, x->rows,
                                    cfg_.EffectiveOutputDim());
}

// :1123-1141
TransformerTrainer::MatPtr TransformerTrainer::AttentionForwardWithCache(MultiHeadAttention &attention,
                                                                         const MatPtr &input, bool causal,
                                                                         AttentionCache &cache) {
  const int seqLen = input->rows, D = cfg_.EmbeddingDim, H = cfg_.NumHeads;
  auto qkv = accel_->ProjectQKV(*input, attention.WQ, attention.BiasQ, attention.WK, attention.BiasK, attention.WV,
                                attention.BiasV);
  auto Q = std::make_shared<Matrix>(std::move(std::get<0>(qkv)));
  auto K = std::make_shared<Matrix>(std::move(std::get<1>(qkv)));
  auto V = std::make_shared<Matrix>(std::move(std::get<2>(qkv)));
  // RotaryPositionEmbedding.ApplyInPlace(q, k, numHeads) (RotaryPositionEmbedding.cs:21-52)
  accel_->ApplyRotaryPositionEmbeddingInPlace(ref(*Q), H, 10000.0f, false);
  accel_->ApplyRotaryPositionEmbeddingInPlace(ref(*K), H, 10000.0f, false);
  cache.Q = Q;
  cache.K = K;
  cache.V = V;
  auto concatenated = std::make_shared<Matrix>(accel_->ScaledDotProductAttention(*Q, *K, *V, H, MaskView{}, causal));
  cache.AttentionOutput = concatenated;
  return std::make_shared<Matrix>(
      accel_->ProjectOutputBatch(*concatenated, attention.WO, attention.BiasO, seqLen, D));
}

// :723-809, the inline attention and RoPE on the manager's capabilities
TransformerTrainer::MatPtr TransformerTrainer::SegmentedAttentionForwardWithCache(
    MultiHeadAttention &attention, const MatPtr &input, int segmentLength, int segmentCount, bool causal,
    AttentionCache &cache) {
  const int totalRows = input->rows, D = cfg_.EmbeddingDim, H = cfg_.NumHeads;
  if (segmentLength <= 0 || segmentCount <= 0 || totalRows != segmentLength * segmentCount)
    throw ArgumentException("Invalid segmented attention shape.");
  auto qkv = accel_->ProjectQKV(*input, attention.WQ, attention.BiasQ, attention.WK, attention.BiasK, attention.WV,
                                attention.BiasV);
  auto Q = std::make_shared<Matrix>(std::move(std::get<0>(qkv)));
  auto K = std::make_shared<Matrix>(std::move(std::get<1>(qkv)));
  auto V = std::make_shared<Matrix>(std::move(std::get<2>(qkv)));
  accel_->ApplySegmentedRotaryInPlace(ref(*Q), ref(*K), H, segmentLength, false);
  auto concatenated =
      std::make_shared<Matrix>(accel_->SegmentedAttentionForward(*Q, *K, *V, H, segmentLength, segmentCount, causal));
  cache.Q = Q;
  cache.K = K;
  cache.V = V;
  cache.AttentionOutput = concatenated;
  cache.IsSegmented = true;
  cache.SegmentLength = segmentLength;
  cache.SegmentCount = segmentCount;
  cache.Causal = causal;
  return std::make_shared<Matrix>(
      accel_->ProjectOutputBatch(*concatenated, attention.WO, attention.BiasO, totalRows, D));
}

// ---- backward (:874-987) ---------------------------------------------------------
void TransformerTrainer::BackpropFromOutput(Matrix &dOutput, ForwardCache &cache) {
  Matrix dX = accel_->BackpropOutputProjection(dOutput, *cache.FinalHiddenStates, model_.OutputProjection,
                                               ref(grads_.OutputProjectionGrad), ref(grads_.OutputBiasGrad),
                                               dOutput.rows, cfg_.EffectiveOutputDim(), cfg_.EmbeddingDim);
  for (int layer = cfg_.NumLayers - 1; layer >= 0; --layer) dX = BackpropBlock(layer, dX, cache);
  // BackpropInput (:887-896)
  if (!cfg_.UsesDiscreteTokens) {
    accel_->BackpropInputProjection(dX, cache.ContinuousInput, cache.ContinuousInputRowStart,
                                    ref(grads_.InputProjectionGrad), ref(grads_.InputProjectionBiasGrad), dX.rows,
                                    cfg_.EmbeddingDim, cfg_.InputFeatureDim);
    return;
  }
  // MarkTokenRows, then the embedding gradient
  for (int i = 0; i < dX.rows; ++i) {
    const int row = cache.TokenIds[cache.TokenStart + i];
    if ((unsigned)row >= (unsigned)cfg_.VocabSize)
      throw ArgumentOutOfRangeException("row", "Sparse gradient row is outside the vocabulary.");
    if (!grads_.marked[row]) {
      grads_.marked[row] = 1;
      grads_.rows.push_back(row);
    }
  }
  accel_->AccumulateTokenEmbeddingGrad(ref(grads_.TokenEmbeddingGrad), dX, cache.TokenIds, cache.TokenStart, dX.rows,
                                       dX.cols);
}

Matrix TransformerTrainer::BackpropBlock(int layer, Matrix &dOut, ForwardCache &cache) {
  TransformerBlock &block = model_.Blocks[layer];
  LayerNormCache &ln2 = cache.LN2Caches[layer];
  auto b2 = accel_->LayerNormBackward(dOut, *ln2.Normalized, block.LN2Gamma, *ln2.Input, ln2.Mean, ln2.Variance);
  Matrix &dFFResidual = std::get<0>(b2);
  accel_->VectorAccumulate(ref(grads_.LN2Grads[layer].GammaGrad), std::get<1>(b2));
  accel_->VectorAccumulate(ref(grads_.LN2Grads[layer].BetaGrad), std::get<2>(b2));
  // BackpropFFN (:923-931): FeedForwardNetwork.ComputeInputGradientBatch
  std::vector<MatRef> wg;
  std::vector<VecRef> bg;
  for (Matrix &m : ffnWeightGrads_[layer]) wg.push_back(ref(m));
  for (std::vector<float> &v : ffnBiasGrads_[layer]) bg.push_back(ref(v));
  Matrix dNormed1 = accel_->FFNInputGradientBatch(*cache.FFNInputs[layer], dFFResidual, block.FeedForward, wg, bg);
  accel_->MatrixAddInPlace(ref(dNormed1), dFFResidual);
  LayerNormCache &ln1 = cache.LN1Caches[layer];
  auto b1 = accel_->LayerNormBackward(dNormed1, *ln1.Normalized, block.LN1Gamma, *ln1.Input, ln1.Mean, ln1.Variance);
  Matrix &dAttnResidual = std::get<0>(b1);
  accel_->VectorAccumulate(ref(grads_.LN1Grads[layer].GammaGrad), std::get<1>(b1));
  accel_->VectorAccumulate(ref(grads_.LN1Grads[layer].BetaGrad), std::get<2>(b1));
  Matrix dX = BackpropAttention(layer, dAttnResidual, cache.AttentionCaches[layer]);
  accel_->MatrixAddInPlace(ref(dX), dAttnResidual);
  return dX;
}

// :933-987
Matrix TransformerTrainer::BackpropAttention(int layer, Matrix &dOut, AttentionCache &cache) {
  MultiHeadAttention &attention = model_.Blocks[layer].Attention;
  AttentionGradients &g = grads_.AttentionGrads[layer];
  const int seqLen = dOut.rows, D = cfg_.EmbeddingDim, H = cfg_.NumHeads, headDim = D / H;
  Matrix dConcatenated(seqLen, D);
  accel_->BackpropLinearProjection(*cache.AttentionOutput, dOut, attention.WO, ref(g.WO_Grad), ref(g.BiasO_Grad),
                                   ref(dConcatenated));
  const float scale = 1.0f / std::sqrt((float)headDim);
  std::tuple<Matrix, Matrix, Matrix> back;
  if (cache.IsSegmented)
    back = accel_->SegmentedMultiHeadAttentionBackward(*cache.Q, *cache.K, *cache.V, dConcatenated, H, scale,
                                                       cache.SegmentLength, cache.SegmentCount, cache.Causal);
  else if (cfg_.UseDecoderOnly)
    back = accel_->MultiHeadAttentionBackward(*cache.Q, *cache.K, *cache.V, dConcatenated, H, scale, true);
  else
    back = accel_->MultiHeadAttentionBackward(*cache.Q, *cache.K, *cache.V, dConcatenated, H, scale, MaskView{});
  Matrix &dQ = std::get<0>(back), &dK = std::get<1>(back), &dV = std::get<2>(back);
  if (cache.IsSegmented) {
    accel_->ApplySegmentedRotaryInPlace(ref(dQ), ref(dK), H, cache.SegmentLength, true);
  } else {  // RotaryPositionEmbedding.ApplyBackwardInPlace (RotaryPositionEmbedding.cs:74-126)
    accel_->ApplyRotaryPositionEmbeddingInPlace(ref(dQ), H, 10000.0f, true);
    accel_->ApplyRotaryPositionEmbeddingInPlace(ref(dK), H, 10000.0f, true);
  }
  return accel_->BackpropQKV(*cache.Input, dQ, dK, dV, attention.WQ, attention.WK, attention.WV, ref(g.WQ_Grad),
                             ref(g.BiasQ_Grad), ref(g.WK_Grad), ref(g.BiasK_Grad), ref(g.WV_Grad),
                             ref(g.BiasV_Grad));
}

// ---- gradients, norm, clipping, update (:1269-1394) --------------------------------
void TransformerTrainer::ZeroAllGradients() {
  // TransformerGradients.Zero (TransformerGradients.cs:79-105): host loops
  const int D = cfg_.EmbeddingDim;
  for (int row : grads_.rows) {
    std::fill(grads_.TokenEmbeddingGrad.data.begin() + (size_t)row * D,
              grads_.TokenEmbeddingGrad.data.begin() + (size_t)(row + 1) * D, 0.f);
    grads_.marked[row] = 0;
  }
  grads_.rows.clear();
  std::fill(grads_.InputProjectionGrad.data.begin(), grads_.InputProjectionGrad.data.end(), 0.f);
  std::fill(grads_.InputProjectionBiasGrad.begin(), grads_.InputProjectionBiasGrad.end(), 0.f);
  for (AttentionGradients &a : grads_.AttentionGrads) {
    for (Matrix *m : {&a.WQ_Grad, &a.WK_Grad, &a.WV_Grad, &a.WO_Grad}) std::fill(m->data.begin(), m->data.end(), 0.f);
    for (std::vector<float> *v : {&a.BiasQ_Grad, &a.BiasK_Grad, &a.BiasV_Grad, &a.BiasO_Grad})
      std::fill(v->begin(), v->end(), 0.f);
  }
  for (auto *list : {&grads_.LN1Grads, &grads_.LN2Grads})
    for (LayerNormGradients &l : *list) {
      std::fill(l.GammaGrad.begin(), l.GammaGrad.end(), 0.f);
      std::fill(l.BetaGrad.begin(), l.BetaGrad.end(), 0.f);
    }
  std::fill(grads_.OutputProjectionGrad.data.begin(), grads_.OutputProjectionGrad.data.end(), 0.f);
  std::fill(grads_.OutputBiasGrad.begin(), grads_.OutputBiasGrad.end(), 0.f);
  // the FFN gradients through the manager (:1382-1394)
  for (int layer = 0; layer < cfg_.NumLayers; ++layer) {
    for (Matrix &wg : ffnWeightGrads_[layer]) accel_->ZeroMatrix(ref(wg));
    for (std::vector<float> &bg : ffnBiasGrads_[layer]) accel_->ZeroVector(ref(bg));
  }
}

void TransformerTrainer::ScaleGradients(float scale) {  // :1354-1380
  const int D = cfg_.EmbeddingDim;
  if (cfg_.UsesDiscreteTokens) {
    for (int row : grads_.rows)  // SparseRowGradientTracker.Scale, host loop
      for (int c = 0; c < D; ++c) grads_.TokenEmbeddingGrad.at(row, c) *= scale;
  } else {
    accel_->MatrixScaleInPlace(ref(grads_.InputProjectionGrad), scale);
    accel_->VectorScaleInPlace(ref(grads_.InputProjectionBiasGrad), scale);
  }
  accel_->MatrixScaleInPlace(ref(grads_.OutputProjectionGrad), scale);
  accel_->VectorScaleInPlace(ref(grads_.OutputBiasGrad), scale);
  for (AttentionGradients &g : grads_.AttentionGrads) {
    accel_->MatrixScaleInPlace(ref(g.WQ_Grad), scale);
    accel_->MatrixScaleInPlace(ref(g.WK_Grad), scale);
    accel_->MatrixScaleInPlace(ref(g.WV_Grad), scale);
    accel_->MatrixScaleInPlace(ref(g.WO_Grad), scale);
    accel_->VectorScaleInPlace(ref(g.BiasQ_Grad), scale);
    accel_->VectorScaleInPlace(ref(g.BiasK_Grad), scale);
    accel_->VectorScaleInPlace(ref(g.BiasV_Grad), scale);
    accel_->VectorScaleInPlace(ref(g.BiasO_Grad), scale);
  }
  for (auto *list : {&grads_.LN1Grads, &grads_.LN2Grads})
    for (LayerNormGradients &l : *list) {
      accel_->VectorScaleInPlace(ref(l.GammaGrad), scale);
      accel_->VectorScaleInPlace(ref(l.BetaGrad), scale);
    }
  for (int layer = 0; layer < cfg_.NumLayers; ++layer) {
    for (Matrix &wg : ffnWeightGrads_[layer]) accel_->MatrixScaleInPlace(ref(wg), scale);
    for (std::vector<float> &bg : ffnBiasGrads_[layer]) accel_->VectorScaleInPlace(ref(bg), scale);
  }
}

float TransformerTrainer::ComputeGradientNorm() {  // :1319-1352
  const int D = cfg_.EmbeddingDim;
  float sum = 0.f;
  if (cfg_.UsesDiscreteTokens) {
    float emb = 0.f;  // SparseRowGradientTracker.SquaredNorm: touched rows in first-use order, host loop
    for (int row : grads_.rows)
      for (int c = 0; c < D; ++c) {
        const float v = grads_.TokenEmbeddingGrad.at(row, c);
        emb += v * v;
      }
    sum += emb;
  } else {
    sum += accel_->MatrixSquaredNorm(grads_.InputProjectionGrad);
    sum += accel_->VectorSquaredNorm(grads_.InputProjectionBiasGrad);
  }
  sum += accel_->MatrixSquaredNorm(grads_.OutputProjectionGrad);
  sum += accel_->VectorSquaredNorm(grads_.OutputBiasGrad);
  for (AttentionGradients &g : grads_.AttentionGrads) {
    sum += accel_->MatrixSquaredNorm(g.WQ_Grad) + accel_->MatrixSquaredNorm(g.WK_Grad) +
           accel_->MatrixSquaredNorm(g.WV_Grad) + accel_->MatrixSquaredNorm(g.WO_Grad);
    sum += accel_->VectorSquaredNorm(g.BiasQ_Grad) + accel_->VectorSquaredNorm(g.BiasK_Grad) +
           accel_->VectorSquaredNorm(g.BiasV_Grad) + accel_->VectorSquaredNorm(g.BiasO_Grad);
  }
  for (LayerNormGradients &l : grads_.LN1Grads)
    sum += accel_->VectorSquaredNorm(l.GammaGrad) + accel_->VectorSquaredNorm(l.BetaGrad);
  for (LayerNormGradients &l : grads_.LN2Grads)
    sum += accel_->VectorSquaredNorm(l.GammaGrad) + accel_->VectorSquaredNorm(l.BetaGrad);
  for (int layer = 0; layer < cfg_.NumLayers; ++layer) {
    for (Matrix &wg : ffnWeightGrads_[layer]) sum += accel_->MatrixSquaredNorm(wg);
    for (std::vector<float> &bg : ffnBiasGrads_[layer]) sum += accel_->VectorSquaredNorm(bg);
  }
  return std::sqrt(sum);
}

void TransformerTrainer::ClipGradients(float threshold, float totalNorm) {  // :1311-1317
  if (threshold <= 0.f || std::isnan(threshold) || std::isinf(threshold))
    throw ArgumentOutOfRangeException("threshold", "Gradient clip threshold must be finite and positive.");
  if (is_finite(totalNorm) && totalNorm > threshold) ScaleGradients(threshold / totalNorm);
}

void TransformerTrainer::UpdateParameters(float learningRate) {  // :1269-1305
  const int D = cfg_.EmbeddingDim;
  if (cfg_.UsesDiscreteTokens) {
    for (int row : grads_.rows)  // SparseRowGradientTracker.UpdateRows, host loop
      for (int c = 0; c < D; ++c)
        model_.TokenEmbedding.at(row, c) -= learningRate * grads_.TokenEmbeddingGrad.at(row, c);
  } else {
    accel_->MatrixUpdate(ref(model_.InputProjection), grads_.InputProjectionGrad, learningRate);
    accel_->VectorUpdate(ref(model_.InputProjectionBias), grads_.InputProjectionBiasGrad, learningRate);
  }
  for (int i = 0; i < cfg_.NumLayers; ++i) {
    TransformerBlock &block = model_.Blocks[i];
    AttentionGradients &g = grads_.AttentionGrads[i];
    accel_->MatrixUpdate(ref(block.Attention.WQ), g.WQ_Grad, learningRate);
    accel_->MatrixUpdate(ref(block.Attention.WK), g.WK_Grad, learningRate);
    accel_->MatrixUpdate(ref(block.Attention.WV), g.WV_Grad, learningRate);
    accel_->MatrixUpdate(ref(block.Attention.WO), g.WO_Grad, learningRate);
    accel_->VectorUpdate(ref(block.Attention.BiasQ), g.BiasQ_Grad, learningRate);
    accel_->VectorUpdate(ref(block.Attention.BiasK), g.BiasK_Grad, learningRate);
    accel_->VectorUpdate(ref(block.Attention.BiasV), g.BiasV_Grad, learningRate);
    accel_->VectorUpdate(ref(block.Attention.BiasO), g.BiasO_Grad, learningRate);
    accel_->VectorUpdate(ref(block.LN1Gamma), grads_.LN1Grads[i].GammaGrad, learningRate);
    accel_->VectorUpdate(ref(block.LN1Beta), grads_.LN1Grads[i].BetaGrad, learningRate);
    accel_->VectorUpdate(ref(block.LN2Gamma), grads_.LN2Grads[i].GammaGrad, learningRate);
    accel_->VectorUpdate(ref(block.LN2Beta), grads_.LN2Grads[i].BetaGrad, learningRate);
    // FeedForwardNetwork.ApplyExternalGradients (NeuralNetwork.cs:1004-1019)
    FeedForwardNetwork &f = block.FeedForward;
    for (size_t l = 0; l < f.weights.size(); ++l) {
      accel_->MatrixUpdate(ref(f.weights[l]), ffnWeightGrads_[i][l], learningRate);
      accel_->VectorUpdate(ref(f.biases[l]), ffnBiasGrads_[i][l], learningRate);
    }
  }
  accel_->MatrixUpdate(ref(model_.OutputProjection), grads_.OutputProjectionGrad, learningRate);
  accel_->VectorUpdate(ref(model_.OutputBias), grads_.OutputBiasGrad, learningRate);
}

}  // namespace cdml_host
