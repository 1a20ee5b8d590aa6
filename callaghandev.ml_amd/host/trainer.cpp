// DeviceTrainer: TransformerTrainer for decoder-only token models on the
// device (Transformers/MultiTypeTransformer/TransformerTrainer.cs), built on
// the C ABI of include/cdml.h.  The step follows TrainBatchDiscrete
// (:217-327): ZeroAllGradients, then per length bucket a forward pass with
// cache (:540-622; segmented per sequence :723-848), the cross-entropy
// gradient over the next-token targets (:660-674) scaled by the bucket size
// when it holds more than one sequence (:291-294), and the backward pass
// (:874-987); then the 1/validCount scale, the global norm, clipping and the
// SGD update (:311-327, :1269-1384).  Nothing here computes on the CPU beyond
// bucketing token ids.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>

#include "cdml_host.h"

namespace cdml_host {

namespace {

void check(int rc, const char *what) {
  if (rc != CDML_OK)
    throw InvalidOperationException(std::string(what) + ": " + cdml_last_error());
}

size_t round64(size_t n) { return (n + 63) / 64 * 64; }  // 256-byte aligned tensors

// Hidden FFN activations whose output alone gives the derivative: the layer
// keeps no pre-activation (cdml_linear_preact with z = NULL).
bool from_output(int act) { return act == Relu || act == Leakyrelu; }

}  // namespace

float *DeviceTrainer::alloc(size_t floats) {
  void *p = nullptr;
  check(cdml_malloc(&p, std::max<size_t>(floats, 1) * sizeof(float)), "cdml_malloc");
  allocs_.push_back(p);
  return static_cast<float *>(p);
}

DeviceTrainer::DeviceTrainer(const LanguageModel &model, const TrainingConfig &config,
                             int batch_capacity, int seq_capacity, int device)
    : cfg_(model.config()), tc_(config), cap_b_(batch_capacity), cap_s_(seq_capacity),
      device_(device) {
  if (batch_capacity <= 0) throw ArgumentOutOfRangeException("batch_capacity");
  if (seq_capacity <= 0 || seq_capacity > cfg_.MaxSequenceLength)
    throw ArgumentOutOfRangeException("seq_capacity");
  if (tc_.UseGradientClipping && !(tc_.GradientClipThreshold > 0.f && std::isfinite(tc_.GradientClipThreshold)))
    throw ArgumentOutOfRangeException("GradientClipThreshold", "Gradient clip threshold must be finite and positive.");
  check(cdml_init(device), "cdml_init");
  check(cdml_stream_create(&stream_), "cdml_stream_create");
  try {
    const int D = cfg_.EmbeddingDim, H = cfg_.NumHeads, V = cfg_.EffectiveOutputDim(), hd = D / H;
    const int F = cfg_.InputFeatureDim;
    const bool discrete = cfg_.UsesDiscreteTokens;
    // ---- parameter layout: one buffer for the weights, one for the gradients
    struct Spec {
      std::string name;
      const float *host;
      size_t count;
    };
    std::vector<Spec> specs;
    if (discrete) {
      specs.push_back({"token_embedding", model.TokenEmbedding.ptr(), model.TokenEmbedding.data.size()});
    } else {
      specs.push_back({"input_proj", model.InputProjection.ptr(), model.InputProjection.data.size()});
      specs.push_back({"input_bias", model.InputProjectionBias.data(), model.InputProjectionBias.size()});
    }
    specs.push_back({"out_proj", model.OutputProjection.ptr(), model.OutputProjection.data.size()});
    specs.push_back({"out_bias", model.OutputBias.data(), model.OutputBias.size()});
    for (size_t l = 0; l < model.Blocks.size(); ++l) {
      const TransformerBlock &b = model.Blocks[l];
      const MultiHeadAttention &a = b.Attention;
      const std::string p = "layers." + std::to_string(l) + ".";
      specs.push_back({p + "wq", a.WQ.ptr(), a.WQ.data.size()});
      specs.push_back({p + "wk", a.WK.ptr(), a.WK.data.size()});
      specs.push_back({p + "wv", a.WV.ptr(), a.WV.data.size()});
      specs.push_back({p + "wo", a.WO.ptr(), a.WO.data.size()});
      specs.push_back({p + "bq", a.BiasQ.data(), a.BiasQ.size()});
      specs.push_back({p + "bk", a.BiasK.data(), a.BiasK.size()});
      specs.push_back({p + "bv", a.BiasV.data(), a.BiasV.size()});
      specs.push_back({p + "bo", a.BiasO.data(), a.BiasO.size()});
      specs.push_back({p + "ln1_g", b.LN1Gamma.data(), b.LN1Gamma.size()});
      specs.push_back({p + "ln1_b", b.LN1Beta.data(), b.LN1Beta.size()});
      specs.push_back({p + "ln2_g", b.LN2Gamma.data(), b.LN2Gamma.size()});
      specs.push_back({p + "ln2_b", b.LN2Beta.data(), b.LN2Beta.size()});
      for (size_t i = 0; i < b.FeedForward.weights.size(); ++i)
        specs.push_back({p + "ffn_w" + std::to_string(i + 1), b.FeedForward.weights[i].ptr(),
                         b.FeedForward.weights[i].data.size()});
      for (size_t i = 0; i < b.FeedForward.biases.size(); ++i)
        specs.push_back({p + "ffn_b" + std::to_string(i + 1), b.FeedForward.biases[i].data(),
                         b.FeedForward.biases[i].size()});
    }
    std::unordered_map<std::string, size_t> at;
    for (const Spec &s : specs) {
      at[s.name] = offs_.size();
      names_.push_back(s.name);
      offs_.push_back({nparams_, s.count});
      nparams_ += round64(s.count);
    }
    params_ = alloc(nparams_);
    grads_ = alloc(nparams_);
    check(cdml_zero_f32_async(params_, nparams_, stream_), "cdml_zero_f32_async");
    for (size_t i = 0; i < specs.size(); ++i)
      check(cdml_memcpy_h2d_async(params_ + offs_[i].first, specs[i].host, specs[i].count * sizeof(float),
                                  stream_),
            "cdml_memcpy_h2d_async");
    auto W = [&](const std::string &n) { return params_ + offs_[at.at(n)].first; };
    auto G = [&](const std::string &n) { return grads_ + offs_[at.at(n)].first; };
    if (discrete) {
      emb_ = W("token_embedding");
      gemb_ = G("token_embedding");
    } else {
      emb_ = W("input_proj");
      inbias_ = W("input_bias");
      gemb_ = G("input_proj");
      ginbias_ = G("input_bias");
    }
    outproj_ = W("out_proj");
    outbias_ = W("out_bias");
    goutproj_ = G("out_proj");
    goutbias_ = G("out_bias");

    // ---- the cdml_param table in the order and grouping of ComputeGradientNorm
    // (TransformerTrainer.cs:1319-1352)
    std::vector<cdml_param> table;
    int group = 0;
    auto add = [&](const std::string &n, int grp) {
      const size_t i = at.at(n);
      table.push_back(cdml_param{params_ + offs_[i].first, grads_ + offs_[i].first,
                                 (long long)offs_[i].second, grp, 0});
    };
    if (discrete) {
      add("token_embedding", group++);
    } else {  // InputProjectionGrad and its bias, two terms (:1327-1328)
      add("input_proj", group++);
      add("input_bias", group++);
    }
    add("out_proj", group++);
    add("out_bias", group++);
    const int L = (int)model.Blocks.size();
    for (int l = 0; l < L; ++l) {
      const std::string p = "layers." + std::to_string(l) + ".";
      for (const char *k : {"wq", "wk", "wv", "wo"}) add(p + k, group);
      ++group;
      for (const char *k : {"bq", "bk", "bv", "bo"}) add(p + k, group);
      ++group;
    }
    for (const char *ln : {"ln1", "ln2"})
      for (int l = 0; l < L; ++l) {
        const std::string p = "layers." + std::to_string(l) + "." + ln;
        add(p + "_g", group);
        add(p + "_b", group);
        ++group;
      }
    for (int l = 0; l < L; ++l) {
      const FeedForwardNetwork &f = model.Blocks[l].FeedForward;
      const std::string p = "layers." + std::to_string(l) + ".";
      for (size_t i = 0; i < f.weights.size(); ++i) add(p + "ffn_w" + std::to_string(i + 1), group++);
      for (size_t i = 0; i < f.biases.size(); ++i) add(p + "ffn_b" + std::to_string(i + 1), group++);
    }
    param_count_ = (int)table.size();
    void *pt = nullptr;
    check(cdml_malloc(&pt, table.size() * sizeof(cdml_param)), "cdml_malloc");
    allocs_.push_back(pt);
    param_table_ = pt;
    check(cdml_memcpy_h2d_async(pt, table.data(), table.size() * sizeof(cdml_param), stream_),
          "cdml_memcpy_h2d_async");

    // ---- per-layer pointers and the forward cache
    const size_t rows = (size_t)cap_b_ * cap_s_;
    int ffmax = D;
    for (int l = 0; l < L; ++l) {
      const TransformerBlock &b = model.Blocks[l];
      const std::string p = "layers." + std::to_string(l) + ".";
      Layer Y{};
      Y.wq = W(p + "wq"); Y.wk = W(p + "wk"); Y.wv = W(p + "wv"); Y.wo = W(p + "wo");
      Y.bq = W(p + "bq"); Y.bk = W(p + "bk"); Y.bv = W(p + "bv"); Y.bo = W(p + "bo");
      Y.ln1g = W(p + "ln1_g"); Y.ln1b = W(p + "ln1_b"); Y.ln2g = W(p + "ln2_g"); Y.ln2b = W(p + "ln2_b");
      Y.gwq = G(p + "wq"); Y.gwk = G(p + "wk"); Y.gwv = G(p + "wv"); Y.gwo = G(p + "wo");
      Y.gbq = G(p + "bq"); Y.gbk = G(p + "bk"); Y.gbv = G(p + "bv"); Y.gbo = G(p + "bo");
      Y.gln1g = G(p + "ln1_g"); Y.gln1b = G(p + "ln1_b"); Y.gln2g = G(p + "ln2_g"); Y.gln2b = G(p + "ln2_b");
      int width = D;
      const FeedForwardNetwork &f = b.FeedForward;
      if (f.weights.empty()) throw InvalidOperationException("Neural network must have at least input and output layers.");
      for (size_t i = 0; i < f.weights.size(); ++i) {
        if (f.weights[i].cols != width) throw ArgumentException("FFN layer widths do not chain.");
        Y.ffw.push_back(W(p + "ffn_w" + std::to_string(i + 1)));
        Y.ffb.push_back(W(p + "ffn_b" + std::to_string(i + 1)));
        Y.gffw.push_back(G(p + "ffn_w" + std::to_string(i + 1)));
        Y.gffb.push_back(G(p + "ffn_b" + std::to_string(i + 1)));
        Y.ffrows.push_back(f.weights[i].rows);
        Y.ffcols.push_back(f.weights[i].cols);
        Y.ffact.push_back(f.activations[i]);
        width = f.weights[i].rows;
        if (i + 1 < f.weights.size()) {
          // ReLU and leaky ReLU layers keep only their output: it carries
          // the derivative (CDML_ACT_FROM_OUTPUT)
          Y.z.push_back(from_output(f.activations[i]) ? nullptr : alloc(rows * width));
          Y.h.push_back(alloc(rows * width));
          ffmax = std::max(ffmax, width);
        }
      }
      if (width != D) throw ArgumentException("FFN output width must equal EmbeddingDim.");
      if (f.activations.back() != None)  // TransformerBlock's FFN ends linear (TransformerBlock.cs:101-123)
        throw InvalidOperationException("DeviceTrainer needs an FFN whose output layer has no activation.");
      Y.x = alloc(rows * D);
      Y.q = alloc(rows * D);
      Y.k = alloc(rows * D);
      Y.v = alloc(rows * D);
      Y.att = alloc(rows * D);
      Y.r1 = alloc(rows * D);
      Y.n1 = alloc(rows * D);
      Y.r2 = alloc(rows * D);
      Y.m1 = alloc(rows);
      Y.v1 = alloc(rows);
      Y.m2 = alloc(rows);
      Y.v2 = alloc(rows);
      // the saved-statistics attention backward covers head dims up to 128
      Y.lse = hd <= 128 ? alloc((size_t)cap_b_ * H * cap_s_) : nullptr;
      layers_.push_back(std::move(Y));
    }
    xfinal_ = alloc(rows * D);
    logits_ = alloc(rows * (size_t)V);
    for (float **p : {&dx_, &dxa_, &dr1_, &dr2_, &dn1_, &dcat_, &dq_, &dk_, &dv_, &tmp_}) *p = alloc(rows * D);
    dh_.push_back(alloc(rows * ffmax));
    dh_.push_back(alloc(rows * ffmax));
    if (!discrete) {
      inputs_ = alloc(rows * F);
      regt_ = alloc(rows * (size_t)V);
    }
    ids_ = reinterpret_cast<int *>(alloc(rows));
    targets_ = reinterpret_cast<int *>(alloc(rows));
    order_ = reinterpret_cast<int *>(alloc(rows));
    gstart_ = reinterpret_cast<int *>(alloc(rows + 1));
    gtoken_ = reinterpret_cast<int *>(alloc(rows));
    result_ = alloc(4);
    losses_ = alloc(64);
    rope_cs_ = alloc((size_t)cap_s_ * hd);
    check(cdml_rope_table(rope_cs_, cap_s_, hd, 10000.0f, stream_), "cdml_rope_table");
    // one workspace for every call of a step (they run in turn on the stream)
    size_t need = 0, n = 0;
    const int R = (int)rows;
    check(cdml_sdpa_bwd_workspace_size(cap_b_, cap_s_, cap_s_, D, H, &n), "workspace size");
    need = std::max(need, n);
    // room for the stored dS blocks (2 * seq^2 bytes per sequence and head),
    // so that the attention backward forms dQ as one product
    check(cdml_sdpa_bwd_saved_workspace_size(cap_b_, cap_s_, cap_s_, D, H, 1, &n), "workspace size");
    need = std::max(need, n);
    check(cdml_backprop_qkv_workspace_size(R, D, D, &n), "workspace size");
    need = std::max(need, n);
    // the attention output projection (its split need not match Q/K/V's)
    check(cdml_linear_backward_workspace_size(R, D, D, &n), "workspace size");
    need = std::max(need, n);
    check(cdml_linear_backward_workspace_size(R, D, V, &n), "workspace size");
    need = std::max(need, n);
    if (!discrete) {
      check(cdml_linear_backward_workspace_size(R, F, D, &n), "workspace size");
      need = std::max(need, n);
    }
    for (const Layer &Y : layers_)
      for (size_t i = 0; i < Y.ffrows.size(); ++i) {
        check(cdml_linear_backward_workspace_size(R, Y.ffcols[i], Y.ffrows[i], &n), "workspace size");
        need = std::max(need, n);
      }
    check(cdml_layernorm_backward_workspace_size(R, D, &n), "workspace size");
    need = std::max(need, n);
    check(cdml_cross_entropy_workspace_size(R, &n), "workspace size");
    need = std::max(need, n);
    check(cdml_grad_norm_workspace_size(param_count_, &n), "workspace size");
    need = std::max(need, n);
    ws_bytes_ = need;
    ws_ = alloc(need / sizeof(float) + 4);
    zero_grads();
    synchronize();
  } catch (...) {
    for (void *p : allocs_) cdml_free(p);
    cdml_stream_destroy(stream_);
    throw;
  }
}

DeviceTrainer::~DeviceTrainer() {
  cdml_stream_synchronize(stream_);
  for (void *p : allocs_) cdml_free(p);
  cdml_stream_destroy(stream_);
}

void DeviceTrainer::synchronize() {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  check(cdml_stream_synchronize(stream_), "cdml_stream_synchronize");
}

void DeviceTrainer::zero_grads() {
  check(cdml_zero_f32_async(grads_, nparams_, stream_), "cdml_zero_f32_async");
}

// Inputs, next-token targets (BuildDiscreteFlatTargets, :660-674) and the
// embedding gradient's row groups of one bucket.
void DeviceTrainer::upload_bucket(const std::vector<const std::vector<int> *> &seqs, int seqLen) {
  const int B = (int)seqs.size(), rows = B * seqLen;
  std::vector<int> ids(rows), tg(rows);
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < seqLen; ++t) {
      ids[b * seqLen + t] = (*seqs[b])[t];
      tg[b * seqLen + t] = (*seqs[b])[t + 1];
    }
  std::vector<int> order(rows);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](int a, int c) { return ids[a] < ids[c]; });
  std::vector<int> start, token;
  for (int i = 0; i < rows; ++i)
    if (i == 0 || ids[order[i]] != ids[order[i - 1]]) {
      start.push_back(i);
      token.push_back(ids[order[i]]);
    }
  start.push_back(rows);
  ngroups_ = (int)token.size();
  // the host vectors must outlive the copies: synchronise before returning
  check(cdml_memcpy_h2d_async(ids_, ids.data(), rows * sizeof(int), stream_), "upload ids");
  check(cdml_memcpy_h2d_async(targets_, tg.data(), rows * sizeof(int), stream_), "upload targets");
  check(cdml_memcpy_h2d_async(order_, order.data(), rows * sizeof(int), stream_), "upload order");
  check(cdml_memcpy_h2d_async(gstart_, start.data(), start.size() * sizeof(int), stream_), "upload groups");
  check(cdml_memcpy_h2d_async(gtoken_, token.data(), token.size() * sizeof(int), stream_), "upload groups");
  synchronize();
}

// Forward with cache and the loss gradient of one bucket of `batch`
// sequences of seqLen inputs (the loss lands in loss_dev).
void DeviceTrainer::bucket_forward(int batch, int seqLen, float grad_scale, float *loss_dev) {
  const int D = cfg_.EmbeddingDim, H = cfg_.NumHeads, V = cfg_.EffectiveOutputDim(), hd = D / H;
  const int F = cfg_.InputFeatureDim;
  const int rows = batch * seqLen;
  const float scale = 1.0f / std::sqrt((float)hd);  // TransformerTrainer.cs:947
  cdml_stream s = stream_;
  const float eps = 1e-5f;
  // ---- forward (ForwardFromEmbeddingWithCache, :540-590)
  float *x0 = layers_.empty() ? xfinal_ : layers_[0].x;
  if (cfg_.UsesDiscreteTokens)
    check(cdml_embed_tokens(ids_, rows, emb_, cfg_.VocabSize, D, x0, nullptr, s), "cdml_embed_tokens");
  else  // BatchDotProductAddBias(InputProjection, input, bias) (:528, :647)
    check(cdml_linear(inputs_, F, emb_, inbias_, x0, D, rows, F, D, CDML_ACT_NONE, s), "cdml_linear");
  for (size_t l = 0; l < layers_.size(); ++l) {
    Layer &Y = layers_[l];
    float *next = l + 1 < layers_.size() ? layers_[l + 1].x : xfinal_;
    check(cdml_project_qkv_rope(Y.x, Y.wq, Y.bq, Y.wk, Y.bk, Y.wv, Y.bv, Y.q, Y.k, Y.v, rows, D, D, hd,
                                rope_cs_, cap_s_, 0, seqLen, s),
          "cdml_project_qkv_rope");
    if (Y.lse)  // keep the row statistics: the backward then skips its forward pass
      check(cdml_sdpa_fwd_lse(Y.q, D, Y.k, D, Y.v, D, Y.att, D, Y.lse, batch, seqLen, seqLen, D, H, scale, 1,
                              nullptr, s),
            "cdml_sdpa_fwd_lse");
    else
      check(cdml_sdpa_fwd(Y.q, D, Y.k, D, Y.v, D, Y.att, D, batch, seqLen, seqLen, D, H, scale, 1, nullptr, s),
            "cdml_sdpa_fwd");
    check(cdml_linear(Y.att, D, Y.wo, Y.bo, tmp_, D, rows, D, D, CDML_ACT_NONE, s), "cdml_linear");
    check(cdml_residual_layernorm_fwd(Y.x, tmp_, Y.ln1g, Y.ln1b, Y.n1, Y.m1, Y.v1, Y.r1, nullptr, rows, D, eps, s),
          "cdml_residual_layernorm_fwd");
    const float *in = Y.n1;
    for (size_t i = 0; i < Y.ffrows.size(); ++i) {
      const int out = Y.ffrows[i], inw = Y.ffcols[i];
      if (i + 1 < Y.ffrows.size()) {
        check(cdml_linear_preact(in, inw, Y.ffw[i], Y.ffb[i], Y.z[i], Y.h[i], out, rows, inw, out, Y.ffact[i], s),
              "cdml_linear_preact");
        in = Y.h[i];
      } else {
        check(cdml_linear(in, inw, Y.ffw[i], Y.ffb[i], tmp_, out, rows, inw, out, Y.ffact[i], s), "cdml_linear");
      }
    }
    check(cdml_residual_layernorm_fwd(Y.n1, tmp_, Y.ln2g, Y.ln2b, next, Y.m2, Y.v2, Y.r2, nullptr, rows, D, eps, s),
          "cdml_residual_layernorm_fwd");
  }
  check(cdml_linear(xfinal_, D, outproj_, outbias_, logits_, V, rows, D, V, CDML_ACT_NONE, s), "cdml_linear");
  // ---- loss and its gradient, in place over the logits (:270-285, :409-438)
  if (cfg_.UsesDiscreteTokens || cfg_.DataType != 1)
    check(cdml_cross_entropy(logits_, V, targets_, rows, V, rows, grad_scale, 1.0f, loss_dev, logits_, V, ws_,
                             ws_bytes_, s),
          "cdml_cross_entropy");
  else
    check(cdml_mse_loss(logits_, V, regt_, V, rows, V, rows, grad_scale, 1.0f, loss_dev, logits_, V, ws_, ws_bytes_,
                        s),
          "cdml_mse_loss");
}

// Backward of the bucket bucket_forward left in the cache; gradients
// accumulate into grads_.
void DeviceTrainer::bucket_backward(int batch, int seqLen) {
  const int D = cfg_.EmbeddingDim, H = cfg_.NumHeads, V = cfg_.EffectiveOutputDim(), hd = D / H;
  const int F = cfg_.InputFeatureDim;
  const int rows = batch * seqLen;
  const float scale = 1.0f / std::sqrt((float)hd);
  cdml_stream s = stream_;
  const float eps = 1e-5f;
  // ---- backward (BackpropFromOutput, :874-921)
  check(cdml_linear_backward(xfinal_, D, logits_, V, outproj_, dx_, D, goutproj_, goutbias_, rows, D, V, 0, ws_,
                             ws_bytes_, s),
        "cdml_linear_backward");
  const float *ga = dx_, *gb = nullptr;  // upstream gradient of the block output: ga (+ gb)
  for (int l = (int)layers_.size() - 1; l >= 0; --l) {
    Layer &Y = layers_[l];
    // LN2 backward; dGamma / dBeta accumulate (VectorAccumulate)
    check(cdml_layernorm_backward(ga, gb, nullptr, Y.ln2g, Y.r2, Y.m2, Y.v2, dr2_, Y.gln2g, Y.gln2b, rows, D, eps,
                                  1, ws_, ws_bytes_, s),
          "cdml_layernorm_backward");
    // FFN (ComputeInputGradientBatch, NeuralNetwork.cs:773-882) with the
    // residual gradient dr2 added to its input gradient (MatrixAddInPlace)
    const int nf = (int)Y.ffrows.size();
    const float *delta = dr2_;
    for (int i = nf - 1; i >= 0; --i) {
      const float *xin = i > 0 ? Y.h[i - 1] : Y.n1;
      float *dxo = i > 0 ? dh_[i & 1] : dn1_;
      const bool fo = i > 0 && !Y.z[i - 1];  // the layer below kept only its output
      check(cdml_linear_backward_act(xin, Y.ffcols[i], delta, Y.ffrows[i], Y.ffw[i],
                                     i > 0 ? (fo ? Y.h[i - 1] : Y.z[i - 1]) : nullptr,
                                     i > 0 ? Y.ffact[i - 1] | (fo ? CDML_ACT_FROM_OUTPUT : 0) : CDML_ACT_NONE, i > 0 ? nullptr : dr2_, dxo,
                                     Y.ffcols[i], Y.gffw[i], Y.gffb[i], rows, Y.ffcols[i], Y.ffrows[i], ws_,
                                     ws_bytes_, s),
            "cdml_linear_backward_act");
      delta = dxo;
    }
    // LN1 backward
    check(cdml_layernorm_backward(dn1_, nullptr, nullptr, Y.ln1g, Y.r1, Y.m1, Y.v1, dr1_, Y.gln1g, Y.gln1b, rows,
                                  D, eps, 1, ws_, ws_bytes_, s),
          "cdml_layernorm_backward");
    // attention (BackpropAttention, :933-987)
    check(cdml_linear_backward(Y.att, D, dr1_, D, Y.wo, dcat_, D, Y.gwo, Y.gbo, rows, D, D, 0, ws_, ws_bytes_, s),
          "cdml_linear_backward");
    // and the inverse rotation of dQ and dK (:978-985), as the kernels store them
    if (Y.lse) {
      check(cdml_sdpa_bwd_saved_rope(Y.q, D, Y.k, D, Y.v, D, Y.att, D, Y.lse, dcat_, D, dq_, D, dk_, D, dv_, D,
                                     batch, seqLen, seqLen, D, H, scale, 1, nullptr, rope_cs_, cap_s_, ws_,
                                     ws_bytes_, s),
            "cdml_sdpa_bwd_saved_rope");
    } else {
      check(cdml_sdpa_bwd(Y.q, D, Y.k, D, Y.v, D, dcat_, D, dq_, D, dk_, D, dv_, D, batch, seqLen, seqLen, D, H,
                          scale, 1, nullptr, ws_, ws_bytes_, s),
            "cdml_sdpa_bwd");
      check(cdml_rope_qk_table(dq_, dk_, rows, D, hd, H, rope_cs_, cap_s_, 0, seqLen, 1, s), "cdml_rope_qk_table");
    }
    check(cdml_backprop_qkv(Y.x, dq_, dk_, dv_, Y.wq, Y.wk, Y.wv, Y.gwq, Y.gbq, Y.gwk, Y.gbk, Y.gwv, Y.gbv, dxa_,
                            rows, D, D, ws_, ws_bytes_, s),
          "cdml_backprop_qkv");
    ga = dxa_;  // dX = dX_attn + dAttnResidual (:919)
    gb = dr1_;
  }
  // BackpropInput (:887-896): the embedding rows of the bucket's tokens, or
  // the input projection (BackpropInputProjection, AccelerationCPU.cs:2280-2332)
  if (cfg_.UsesDiscreteTokens) {
    check(cdml_embedding_grad(gemb_, ga, gb, D, order_, gstart_, gtoken_, ngroups_, D, s), "cdml_embedding_grad");
  } else {
    if (gb) check(cdml_add_inplace(const_cast<float *>(ga), gb, (size_t)rows * D, s), "cdml_add_inplace");
    check(cdml_linear_backward(inputs_, F, ga, D, emb_, nullptr, F, gemb_, ginbias_, rows, F, D, 0, ws_, ws_bytes_,
                               s),
          "cdml_linear_backward");
  }
}

void DeviceTrainer::update(int validCount, float learningRate) {
  const float prescale = 1.0f / (float)validCount;  // ScaleGradients(1.0f / validCount), :313
  check(cdml_grad_norm(static_cast<const cdml_param *>(param_table_), param_count_, prescale,
                       tc_.UseGradientClipping ? 1 : 0, tc_.GradientClipThreshold, result_, ws_, ws_bytes_,
                       stream_),
        "cdml_grad_norm");
  check(cdml_sgd_update(static_cast<const cdml_param *>(param_table_), param_count_, learningRate, prescale,
                        result_, 0, stream_),
        "cdml_sgd_update");
}

// Inputs and targets of one continuous bucket: window rows [0, S) are the
// inputs, rows [1, S] the targets (BuildContinuousRegressionFlatTargets /
// BuildContinuousClassFlatTargets, TransformerTrainer.cs:676-708).
void DeviceTrainer::upload_bucket_continuous(const std::vector<Matrix> &inputs,
                                             const std::vector<Matrix> &regTargets,
                                             const std::vector<std::vector<int>> &classTargets,
                                             const std::vector<int> &idx, int seqLen) {
  const int F = cfg_.InputFeatureDim, O = cfg_.EffectiveOutputDim();
  const int B = (int)idx.size(), rows = B * seqLen;
  std::vector<float> x((size_t)rows * F);
  for (int b = 0; b < B; ++b)
    std::memcpy(x.data() + (size_t)b * seqLen * F, inputs[idx[b]].ptr(), (size_t)seqLen * F * sizeof(float));
  check(cdml_memcpy_h2d_async(inputs_, x.data(), x.size() * sizeof(float), stream_), "upload inputs");
  std::vector<float> rt;
  std::vector<int> ct;
  if (cfg_.DataType == 1) {
    rt.resize((size_t)rows * O);
    for (int b = 0; b < B; ++b)
      std::memcpy(rt.data() + (size_t)b * seqLen * O, regTargets[idx[b]].ptr() + O, (size_t)seqLen * O * sizeof(float));
    check(cdml_memcpy_h2d_async(regt_, rt.data(), rt.size() * sizeof(float), stream_), "upload targets");
  } else {
    ct.resize(rows);
    for (int b = 0; b < B; ++b)
      for (int t = 0; t < seqLen; ++t) ct[b * seqLen + t] = classTargets[idx[b]][t + 1];
    check(cdml_memcpy_h2d_async(targets_, ct.data(), ct.size() * sizeof(int), stream_), "upload targets");
  }
  synchronize();  // the host vectors must outlive the copies
}

float DeviceTrainer::TrainBatchContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> &regTargets,
                                          const std::vector<std::vector<int>> &classTargets, float learningRate) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  if (cfg_.UsesDiscreteTokens) throw InvalidOperationException("Use TrainBatch for token models.");
  const bool regression = cfg_.DataType == 1;
  const int F = cfg_.InputFeatureDim, O = cfg_.EffectiveOutputDim();
  std::vector<int> lens;
  std::unordered_map<int, std::vector<int>> buckets;
  for (size_t i = 0; i < inputs.size(); ++i) {  // the skips of :353-377 and :1480-1502
    const Matrix &x = inputs[i];
    const int T = x.rows;
    if (T < 2 || x.cols != F) continue;
    bool ok = std::all_of(x.data.begin(), x.data.end(), [](float v) { return std::isfinite(v); });
    if (regression) {
      ok = ok && i < regTargets.size() && regTargets[i].rows >= T && regTargets[i].cols == O &&
           std::all_of(regTargets[i].data.begin(), regTargets[i].data.end(), [](float v) { return std::isfinite(v); });
    } else {
      ok = ok && i < classTargets.size() && (int)classTargets[i].size() >= T;
      for (int t = 1; ok && t < T; ++t) ok = (unsigned)classTargets[i][t] < (unsigned)O;
    }
    if (!ok) continue;
    if (!buckets.count(T - 1)) lens.push_back(T - 1);
    buckets[T - 1].push_back((int)i);
  }
  loaded_b_ = 0;
  zero_grads();
  float totalLoss = 0.f;
  int validCount = 0;
  for (int inputLen : lens) {
    const auto &all = buckets[inputLen];
    if (inputLen > cap_s_) throw ArgumentOutOfRangeException("inputs", "window longer than the trainer's seq_capacity");
    for (size_t start = 0; start < all.size(); start += cap_b_) {
      std::vector<int> part(all.begin() + start, all.begin() + std::min(all.size(), start + cap_b_));
      const int B = (int)part.size();
      upload_bucket_continuous(inputs, regTargets, classTargets, part, inputLen);
      bucket_forward(B, inputLen, B > 1 ? (float)B : 1.0f, losses_);
      float loss = 0.f;
      check(cdml_memcpy_d2h_async(&loss, losses_, sizeof(float), stream_), "read loss");
      synchronize();
      if (!std::isfinite(loss)) continue;
      bucket_backward(B, inputLen);
      totalLoss += loss * B;  // :451
      validCount += B;
    }
  }
  if (validCount == 0) return 0.f;
  update(validCount, learningRate);
  float res[3];
  check(cdml_memcpy_d2h_async(res, result_, sizeof(res), stream_), "read norm");
  synchronize();
  last_norm_ = res[0];
  return totalLoss / validCount;
}

float DeviceTrainer::TrainContinuous(const std::vector<Matrix> &inputs, const std::vector<Matrix> &regTargets,
                                     const std::vector<std::vector<int>> &classTargets, uint64_t seed) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  if (cfg_.UsesDiscreteTokens) throw InvalidOperationException("Use Train(int[][]) for token models.");
  if (tc_.BatchSize <= 0) throw ArgumentOutOfRangeException("BatchSize", "BatchSize must be positive.");
  if (tc_.Epochs < 0) throw ArgumentOutOfRangeException("Epochs", "Epochs must be non-negative.");
  if (cfg_.DataType == 1 && regTargets.size() != inputs.size())
    throw ArgumentException("regressionTargets length must match inputs length.", "regressionTargets");
  if (cfg_.DataType == 2 && classTargets.size() != inputs.size())
    throw ArgumentException("classTargets length must match inputs length.", "classTargets");
  std::vector<int> valid;
  for (size_t i = 0; i < inputs.size(); ++i) {
    if (inputs[i].rows < 2) continue;
    if (inputs[i].cols != cfg_.InputFeatureDim)
      throw ArgumentException("Input sequence " + std::to_string(i) + " has feature dimension " +
                                  std::to_string(inputs[i].cols) + ", expected " +
                                  std::to_string(cfg_.InputFeatureDim) + ".",
                              "inputs");
    valid.push_back((int)i);
  }
  if (valid.empty()) throw ArgumentException("No valid sequences. All must have at least 2 timesteps.", "inputs");
  float lr = tc_.LearningRate, epochAvg = 0.f;
  uint64_t state = seed;
  auto next = [&state]() {  // SplitMix64
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  };
  for (int epoch = 0; epoch < tc_.Epochs; ++epoch) {
    std::vector<int> order = valid;
    for (size_t i = order.size(); i > 1; --i) std::swap(order[i - 1], order[next() % i]);
    float epochLoss = 0.f;
    int numBatches = 0;
    for (size_t i = 0; i < order.size(); i += tc_.BatchSize) {
      std::vector<Matrix> bx;
      std::vector<Matrix> br;
      std::vector<std::vector<int>> bc;
      for (size_t j = i; j < std::min(order.size(), i + (size_t)tc_.BatchSize); ++j) {
        bx.push_back(inputs[order[j]]);
        if (cfg_.DataType == 1) br.push_back(regTargets[order[j]]);
        else bc.push_back(classTargets[order[j]]);
      }
      epochLoss += TrainBatchContinuous(bx, br, bc, lr);
      ++numBatches;
    }
    epochAvg = numBatches > 0 ? epochLoss / numBatches : 0.f;
    if (tc_.UseLearningRateDecay) lr *= tc_.LearningRateDecay;
  }
  return epochAvg;
}

float DeviceTrainer::TrainBatch(const std::vector<std::vector<int>> &batch, float learningRate) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  if (!cfg_.UsesDiscreteTokens) throw InvalidOperationException("Use TrainBatchContinuous for continuous inputs.");
  // TokensAreValid (:1467-1478) and the length buckets (:224-248), in order of
  // first appearance
  std::vector<int> lens;
  std::unordered_map<int, std::vector<const std::vector<int> *>> buckets;
  for (const auto &seq : batch) {
    if (seq.size() < 2) continue;
    bool ok = true;
    for (int t : seq) ok = ok && t >= 0 && t < cfg_.VocabSize;
    if (!ok) continue;
    const int inputLen = (int)seq.size() - 1;
    if (!buckets.count(inputLen)) lens.push_back(inputLen);
    buckets[inputLen].push_back(&seq);
  }
  loaded_b_ = 0;
  zero_grads();  // ZeroAllGradients (:222)
  float totalLoss = 0.f;
  int validCount = 0;
  for (int inputLen : lens) {
    const auto &all = buckets[inputLen];
    if (inputLen > cap_s_) throw ArgumentOutOfRangeException("batch", "sequence longer than the trainer's seq_capacity");
    for (size_t start = 0; start < all.size(); start += cap_b_) {  // buckets beyond the capacity run in parts
      std::vector<const std::vector<int> *> part(all.begin() + start,
                                                 all.begin() + std::min(all.size(), start + cap_b_));
      const int B = (int)part.size();
      upload_bucket(part, inputLen);
      bucket_forward(B, inputLen, B > 1 ? (float)B : 1.0f, losses_);
      float loss = 0.f;
      check(cdml_memcpy_d2h_async(&loss, losses_, sizeof(float), stream_), "read loss");
      synchronize();
      if (!std::isfinite(loss)) continue;  // no backward for this bucket (:273-274, :288-289)
      bucket_backward(B, inputLen);
      totalLoss += B > 1 ? loss * B : loss;
      validCount += B;
    }
  }
  if (validCount == 0) return 0.f;
  update(validCount, learningRate);
  float res[3];
  check(cdml_memcpy_d2h_async(res, result_, sizeof(res), stream_), "read norm");
  synchronize();
  last_norm_ = res[0];
  return totalLoss / validCount;
}

void DeviceTrainer::load_batch(const int *host_tokens, int batch, int seqLenPlus1) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  if (!cfg_.UsesDiscreteTokens) throw InvalidOperationException("load_batch takes token sequences.");
  if (batch <= 0 || batch > cap_b_ || seqLenPlus1 < 2 || seqLenPlus1 - 1 > cap_s_)
    throw ArgumentOutOfRangeException("batch");
  std::vector<std::vector<int>> seqs(batch);
  for (int b = 0; b < batch; ++b) seqs[b].assign(host_tokens + (size_t)b * seqLenPlus1, host_tokens + (size_t)(b + 1) * seqLenPlus1);
  std::vector<const std::vector<int> *> part;
  for (auto &q : seqs) part.push_back(&q);
  for (int i = 0; i < batch * seqLenPlus1; ++i)
    if (host_tokens[i] < 0 || host_tokens[i] >= cfg_.VocabSize) throw ArgumentOutOfRangeException("host_tokens");
  upload_bucket(part, seqLenPlus1 - 1);
  loaded_b_ = batch;
  loaded_s_ = seqLenPlus1 - 1;
}

void DeviceTrainer::load_batch_continuous(const float *host_inputs, const float *host_targets, int batch,
                                          int seqLenPlus1) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  if (cfg_.UsesDiscreteTokens || cfg_.DataType != 1)
    throw InvalidOperationException("load_batch_continuous takes regression windows.");
  if (batch <= 0 || batch > cap_b_ || seqLenPlus1 < 2 || seqLenPlus1 - 1 > cap_s_)
    throw ArgumentOutOfRangeException("batch");
  const int F = cfg_.InputFeatureDim, O = cfg_.EffectiveOutputDim();
  std::vector<Matrix> xs(batch), ts(batch);
  std::vector<int> idx(batch);
  for (int b = 0; b < batch; ++b) {
    xs[b] = Matrix(seqLenPlus1, F);
    ts[b] = Matrix(seqLenPlus1, O);
    std::memcpy(xs[b].ptr(), host_inputs + (size_t)b * seqLenPlus1 * F, (size_t)seqLenPlus1 * F * sizeof(float));
    std::memcpy(ts[b].ptr(), host_targets + (size_t)b * seqLenPlus1 * O, (size_t)seqLenPlus1 * O * sizeof(float));
    idx[b] = b;
  }
  upload_bucket_continuous(xs, ts, {}, idx, seqLenPlus1 - 1);
  loaded_b_ = batch;
  loaded_s_ = seqLenPlus1 - 1;
}

void DeviceTrainer::step_loaded(float learningRate) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  if (loaded_b_ <= 0) throw InvalidOperationException("load_batch first");
  zero_grads();
  bucket_forward(loaded_b_, loaded_s_, loaded_b_ > 1 ? (float)loaded_b_ : 1.0f, losses_);
  bucket_backward(loaded_b_, loaded_s_);
  update(loaded_b_, learningRate);
}

float DeviceTrainer::Train(const std::vector<std::vector<int>> &sequences, uint64_t seed) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  if (!cfg_.UsesDiscreteTokens) throw InvalidOperationException("Use TrainContinuous() for continuous inputs.");
  if (tc_.BatchSize <= 0) throw ArgumentOutOfRangeException("BatchSize", "BatchSize must be positive.");
  if (tc_.Epochs < 0) throw ArgumentOutOfRangeException("Epochs", "Epochs must be non-negative.");
  std::vector<const std::vector<int> *> valid;
  for (const auto &s : sequences)
    if (s.size() >= 2) valid.push_back(&s);
  if (valid.empty())
    throw ArgumentException("No valid sequences to train on. All sequences must contain at least 2 tokens.",
                            "sequences");
  float lr = tc_.LearningRate, epochAvg = 0.f;
  uint64_t state = seed;
  auto next = [&state]() {  // SplitMix64
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  };
  for (int epoch = 0; epoch < tc_.Epochs; ++epoch) {
    std::vector<const std::vector<int> *> order = valid;
    for (size_t i = order.size(); i > 1; --i) std::swap(order[i - 1], order[next() % i]);  // Fisher-Yates
    float epochLoss = 0.f;
    int numBatches = 0;
    for (size_t i = 0; i < order.size(); i += tc_.BatchSize) {
      std::vector<std::vector<int>> b;
      for (size_t j = i; j < std::min(order.size(), i + (size_t)tc_.BatchSize); ++j) b.push_back(*order[j]);
      epochLoss += TrainBatch(b, lr);
      ++numBatches;
    }
    epochAvg = numBatches > 0 ? epochLoss / numBatches : 0.f;
    if (tc_.UseLearningRateDecay) lr *= tc_.LearningRateDecay;
  }
  return epochAvg;
}

std::vector<float> DeviceTrainer::weights_flat() {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  std::vector<float> h(nparams_);
  check(cdml_memcpy_d2h_async(h.data(), params_, nparams_ * sizeof(float), stream_), "download");
  synchronize();
  return h;
}

std::vector<float> DeviceTrainer::gradients_flat() {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  std::vector<float> h(nparams_);
  check(cdml_memcpy_d2h_async(h.data(), grads_, nparams_ * sizeof(float), stream_), "download");
  synchronize();
  return h;
}

void DeviceTrainer::CopyWeightsTo(LanguageModel &model) {
  std::lock_guard<std::recursive_mutex> lock(mu_);
  const std::vector<float> w = weights_flat();
  size_t i = 0;
  auto take = [&](float *dst, size_t n) {
    if (offs_[i].second != n) throw ArgumentException("model shape differs from the trainer's");
    std::memcpy(dst, w.data() + offs_[i].first, n * sizeof(float));
    ++i;
  };
  if (cfg_.UsesDiscreteTokens) {
    take(model.TokenEmbedding.ptr(), model.TokenEmbedding.data.size());
  } else {
    take(model.InputProjection.ptr(), model.InputProjection.data.size());
    take(model.InputProjectionBias.data(), model.InputProjectionBias.size());
  }
  take(model.OutputProjection.ptr(), model.OutputProjection.data.size());
  take(model.OutputBias.data(), model.OutputBias.size());
  for (TransformerBlock &b : model.Blocks) {
    MultiHeadAttention &a = b.Attention;
    for (Matrix *m : {&a.WQ, &a.WK, &a.WV, &a.WO}) take(m->ptr(), m->data.size());
    for (std::vector<float> *v : {&a.BiasQ, &a.BiasK, &a.BiasV, &a.BiasO}) take(v->data(), v->size());
    for (std::vector<float> *v : {&b.LN1Gamma, &b.LN1Beta, &b.LN2Gamma, &b.LN2Beta}) take(v->data(), v->size());
    for (Matrix &m : b.FeedForward.weights) take(m.ptr(), m.data.size());
    for (std::vector<float> &v : b.FeedForward.biases) take(v.data(), v.size());
  }
}

}  // namespace cdml_host
