// cdml_mha_layer_fwd: MultiHeadAttention.Forward of one self-attention layer
// on device buffers in one C-ABI call (MultiHeadAttention.cs:96-111,146-155):
// the fused Q/K/V projection with the rotary embedding of Q and K in its
// epilogue, the flash attention forward, and the output projection.  The
// three launches are the ones a host would chain itself; the entry exists so
// that a managed MultiHeadAttention.Forward override can bind one function.
#include "common.h"

namespace {

constexpr size_t kAlign = 256;

size_t round_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// Workspace layout: q | k | v | attention (rows x dim floats each) | RoPE table
// (seq_len x head_dim floats), each 256-byte aligned.
size_t workspace_bytes(int rows, int dim, int seq_len, int head_dim) {
  const size_t act = round_up((size_t)rows * dim * sizeof(float));
  return 4 * act + round_up((size_t)seq_len * head_dim * sizeof(float));
}

}  // namespace

using namespace cdml;

extern "C" int cdml_mha_layer_fwd_workspace_size(int batch, int seq_len, int dim, int num_heads,
                                                 size_t *bytes) {
  if (!bytes) return fail(CDML_E_INVALID, "cdml_mha_layer_fwd_workspace_size: bytes is NULL");
  if (batch < 0 || seq_len < 0 || dim <= 0 || num_heads <= 0 || dim % num_heads)
    return fail(CDML_E_INVALID, "cdml_mha_layer_fwd_workspace_size: bad size (batch %d, seq_len %d, dim %d, "
                                "heads %d)", batch, seq_len, dim, num_heads);
  if ((int64_t)batch * seq_len > INT32_MAX)
    return fail(CDML_E_INVALID, "cdml_mha_layer_fwd_workspace_size: batch x seq_len = %lld rows exceeds %d",
                (long long)batch * seq_len, INT32_MAX);
  *bytes = workspace_bytes(batch * seq_len, dim, seq_len, dim / num_heads);
  return CDML_OK;
}

extern "C" int cdml_mha_layer_fwd(const float *x, const float *wq, const float *bq, const float *wk,
                                  const float *bk, const float *wv, const float *bv, const float *wo,
                                  const float *bo, float *y, int batch, int seq_len, int dim,
                                  int num_heads, float rope_base, int causal, const uint8_t *mask,
                                  const float *rope_cs, void *workspace, size_t workspace_bytes_,
                                  cdml_stream stream) {
  if (batch < 0 || seq_len < 0 || dim <= 0 || num_heads <= 0)
    return fail(CDML_E_INVALID, "cdml_mha_layer_fwd: bad size (batch %d, seq_len %d, dim %d, heads %d)", batch,
                seq_len, dim, num_heads);
  if (dim % num_heads)
    return fail(CDML_E_INVALID, "cdml_mha_layer_fwd: dim %d not divisible by num_heads %d", dim, num_heads);
  const int head_dim = dim / num_heads;
  if (head_dim & 1) return fail(CDML_E_INVALID, "cdml_mha_layer_fwd: head dim %d must be even (RoPE)", head_dim);
  if ((int64_t)batch * seq_len > INT32_MAX)
    return fail(CDML_E_INVALID, "cdml_mha_layer_fwd: batch x seq_len = %lld rows exceeds %d",
                (long long)batch * seq_len, INT32_MAX);
  if (batch == 0 || seq_len == 0) return CDML_OK;
  if (!x || !wq || !wk || !wv || !wo || !y) return fail(CDML_E_INVALID, "cdml_mha_layer_fwd: NULL pointer");
  const int rows = batch * seq_len;
  const size_t need = workspace_bytes(rows, dim, seq_len, head_dim);
  if (!workspace || workspace_bytes_ < need)
    return fail(CDML_E_INVALID, "cdml_mha_layer_fwd: workspace of %zu bytes, %zu needed", workspace_bytes_, need);
  if (reinterpret_cast<uintptr_t>(workspace) % kAlign)
    return fail(CDML_E_INVALID, "cdml_mha_layer_fwd: workspace must be 256-byte aligned");

  char *ws = static_cast<char *>(workspace);
  const size_t act = round_up((size_t)rows * dim * sizeof(float));
  float *q = reinterpret_cast<float *>(ws);
  float *k = reinterpret_cast<float *>(ws + act);
  float *v = reinterpret_cast<float *>(ws + 2 * act);
  float *att = reinterpret_cast<float *>(ws + 3 * act);
  const float *cs = rope_cs;
  if (!cs) {  // the rotation table of the sequence's positions (MultiHeadAttention.cs:110)
    float *table = reinterpret_cast<float *>(ws + 4 * act);
    int rc = cdml_rope_table(table, seq_len, head_dim, rope_base, stream);
    if (rc) return rc;
    cs = table;
  }
  // ProjectQKV + RoPE of Q and K (:108-110): row r at position r % seq_len
  int rc = cdml_project_qkv_rope(x, wq, bq, wk, bk, wv, bv, q, k, v, rows, dim, dim, head_dim, cs, seq_len, 0,
                                 seq_len, stream);
  if (rc) return rc;
  // ScaledDotProductAttention (:148): scale 1 / sqrt(head_dim), per sequence
  const float scale = 1.0f / sqrtf((float)head_dim);
  rc = cdml_sdpa_fwd(q, dim, k, dim, v, dim, att, dim, batch, seq_len, seq_len, dim, num_heads, scale, causal,
                     mask, stream);
  if (rc) return rc;
  // ProjectOutputBatch (:150-155)
  return cdml_linear(att, dim, wo, bo, y, dim, rows, dim, dim, CDML_ACT_NONE, stream);
}
