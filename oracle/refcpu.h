/*
 * refcpu.h -- CPU parity oracle for the causal multi-head attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a from-scratch C restatement of the
 * CallaghanDev.ML CPU managers (AccelerationCPU, AccelerationMutliThreadCPU)
 * and of the LanguageModel decode/generate flow.  Only tests/, the smoke()
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it, and only as the checker or the timed CPU baseline.  The product path
 * (libcdml_hip.so and the host manager) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the reference repository root, CallaghanDev.ML/...).
 *
 * Conventions (reference: AccelerationCPU.cs, all float[,] are row-major):
 *   matrices are row-major float32 [rows, cols]; weights are [out, in];
 *   masks are uint8 [Lq, Lk] with 1 = attend (bool[,] true = attend).
 * Status codes: 0 ok, -1 invalid argument (the reference throws
 * ArgumentException / ArgumentOutOfRangeException), -2 causal with Lq != Lk.
 */
#ifndef CDML_REFCPU_H
#define CDML_REFCPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Width of System.Numerics.Vector<float> on an AVX2 x86-64 host (32 bytes). */
#define REF_VECTOR_WIDTH 8

/* ---- single-threaded restatement of AccelerationCPU ------------------- */

float ref_dot(const float *a, const float *b, int n);

int ref_project_qkv(const float *x, const float *wq, const float *bq,
                    const float *wk, const float *bk, const float *wv,
                    const float *bv, float *q, float *k, float *v, int rows,
                    int in_dim, int out_dim);

int ref_project_output_batch(const float *h, const float *w, const float *b,
                             float *y, int rows, int in_dim, int out_dim);

int ref_batch_dot_add_bias(const float *w, const float *x, const float *b,
                           float *y, int rows, int in_dim, int out_dim);

void ref_activation_inplace(float *x, long n, int activation);

int ref_rope_inplace(float *x, int rows, int dim, int num_heads,
                     float base_theta, int inverse);

int ref_rope_head_inplace(float *x, int rows, int dim, int start_col,
                          int head_dim, float base_theta, int inverse);

int ref_sdpa(const float *q, const float *k, const float *v, float *out,
             int lq, int lk, int dim, int num_heads, const uint8_t *mask,
             int causal);

int ref_mha_forward(const float *q, const float *k, const float *v, float *out,
                    int lq, int lk, int dim, int num_heads, float scale,
                    const uint8_t *mask);

int ref_softmax(const float *x, float *out, int rows, int cols,
                const uint8_t *mask);

int ref_residual_layernorm(const float *a, const float *b, const float *gamma,
                           const float *beta, float *out, int rows,
                           int features, float eps);

int ref_embed_tokens(const int *ids, int count, const float *table, int vocab,
                     int dim, float *out);

void ref_causal_mask(int n, uint8_t *mask);

/* ---- LanguageModel (decoder-only) flow -------------------------------- */

typedef struct ref_lm_layer {
  const float *wq, *wk, *wv, *wo; /* [D, D] */
  const float *bq, *bk, *bv, *bo; /* [D] */
  const float *ln1_g, *ln1_b;     /* [D] */
  const float *ln2_g, *ln2_b;     /* [D] */
  const float *ffn_w1, *ffn_b1;   /* [FF, D], [FF] */
  const float *ffn_w2, *ffn_b2;   /* [D, FF], [D] */
} ref_lm_layer;

typedef struct ref_lm {
  int vocab, dim, heads, layers, ff, max_seq;
  int ffn_activation;            /* ActivationType of the hidden FFN layer */
  const float *token_embedding;  /* [vocab, D] */
  const float *out_proj;         /* [vocab, D] */
  const float *out_bias;         /* [vocab] */
  const ref_lm_layer *layer;     /* [layers] */
} ref_lm;

int ref_lm_forward(const ref_lm *m, const int *ids, int n, float *logits);
int ref_lm_hidden(const ref_lm *m, const float *embedded, int n, float *hidden);
int ref_lm_generate_greedy(const ref_lm *m, const int *prompt, int n_prompt,
                           int max_new, int *out_tokens, int *out_len);
int ref_decode_attention(const float *q, const float *kcache,
                         const float *vcache, int key_len, int dim,
                         int num_heads, float scale, float *out);

/* ---- backward path (refcpu_bwd.c) -------------------------------------- */

int ref_mha_backward(const float *q, const float *k, const float *v,
                     const float *dout, float *dq, float *dk, float *dv, int lq,
                     int lk, int dim, int num_heads, float scale,
                     const uint8_t *mask, int use_decoder_mask);
int ref_backprop_qkv(const float *x, const float *dq, const float *dk,
                     const float *dv, const float *wq, const float *wk,
                     const float *wv, float *wqg, float *bqg, float *wkg,
                     float *bkg, float *wvg, float *bvg, float *dx, int rows,
                     int in_dim, int out_dim);
int ref_backprop_linear_projection(const float *x, const float *dy,
                                   const float *w, float *wg, float *bg,
                                   float *dx, int rows, int in_dim,
                                   int out_dim);
int ref_backprop_output_projection(const float *dl, const float *x,
                                   const float *w, float *wg, float *bg,
                                   float *dx, int rows, int out_dim,
                                   int emb_dim);

/* ---- training step (refcpu_train.c) ----------------------------------- */

int ref_residual_layernorm_forward(const float *a, const float *b, const float *gamma,
                                   const float *beta, float *out, float *means, float *vars,
                                   float *normalized, float *residual, int rows, int features,
                                   float eps);
int ref_layernorm_backward(const float *dout, const float *normalized, const float *gamma,
                           const float *input, const float *mean, const float *var,
                           float *dinput, float *dgamma, float *dbeta, int rows, int features,
                           float eps);
int ref_cross_entropy(const float *logits, int rows, int out_dim, const int *targets,
                      int n_targets, int target_start, int effective_len, float *loss,
                      float *dlogits);
int ref_ffn_input_gradient(const float *input, const float *dout, int rows, int n_layers,
                           const int *widths, const float *const *w, const float *const *b,
                           const int *act, float *const *wgrad, float *const *bgrad,
                           float *dinput);
int ref_accumulate_token_embedding_grad(float *eg, const float *dx, const int *ids, int n, int dim,
                                        int vocab);
float ref_squared_norm(const float *x, long n);
void ref_scale_inplace(float *x, long n, float scale);
void ref_sgd_update(float *w, const float *g, long n, float lr);
int ref_mse_loss(const float *pred, int rows, int out_dim, const float *targets, int target_rows,
                 int target_start, int effective_len, float *loss, float *dout);
int ref_backprop_input_projection(const float *dx, const float *input, int input_rows,
                                  int input_cols, int row_start, float *wg, float *bg, int seq_len,
                                  int emb_dim, int feat_dim);

/* ---- multi-threaded restatement of AccelerationMutliThreadCPU ---------- */

int mt_num_threads(void);
void mt_set_threads(int n);
int mt_project_qkv(const float *x, const float *wq, const float *bq,
                   const float *wk, const float *bk, const float *wv,
                   const float *bv, float *q, float *k, float *v, int rows,
                   int in_dim, int out_dim);
int mt_project_output_batch(const float *h, const float *w, const float *b,
                            float *y, int rows, int in_dim, int out_dim);
int mt_batch_dot_add_bias(const float *w, const float *x, const float *b,
                          float *y, int rows, int in_dim, int out_dim);
int mt_rope_inplace(float *x, int rows, int dim, int num_heads,
                    float base_theta, int inverse);
int mt_sdpa(const float *q, const float *k, const float *v, float *out, int lq,
            int lk, int dim, int num_heads, const uint8_t *mask, int causal);
int mt_residual_layernorm(const float *a, const float *b, const float *gamma,
                          const float *beta, float *out, int rows,
                          int features, float eps);
int mt_decode_attention_batch(const float *q, const float *kcache,
                              const float *vcache, const int *kv_len,
                              int batch, int t_max, int dim, int num_heads,
                              float scale, float *out, int parallel);

#ifdef __cplusplus
}
#endif

#endif
