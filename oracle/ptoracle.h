/*
 * ptoracle — CPU restatement of pitorch's projection hot path and its
 * neighbours, used ONLY as the parity checker for libptmi.
 *
 * TEST INFRASTRUCTURE.  Nothing in the product (libptmi, libpthost, the
 * pitorch_amd package) links, loads or calls this code.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
 *
 * Every function states the reference file:line it restates (paths are
 * relative to masonwang025/pitorch).  Operation order, literals and
 * int/float conversions follow the reference exactly so that, built with
 * -O2 -ffp-contract=off, results are bit-identical to the reference's own
 * host build (oracle/_ref/libptref.so) — the tests check that.
 *
 * Pinning (how each function is checked beyond the reference build):
 *   math polys .......... test_ops.c KATs (expf/sinf/cosf) + libm bounds
 *   rmsnorm/softmax/... . test_ops.c KATs + fp64 recomputation
 *   po_smatvec .......... test_ops.c 4x6 KAT, integer-exact LCG inputs,
 *                         fp64 brute force with the gamma_n bound
 *   backward ops ........ closed forms (W^T dy, dy x^T), finite differences
 *   po_forward .......... fp64 recomputation of a whole token step, and
 *                         the reference build's pt_forward_step bitwise
 *   po_forward_train .... T x po_forward logits, fp64 loss recompute
 *   po_backward ......... finite differences of po_forward_train's loss
 *   po_sgemm_rect ....... closed form, integer-exact inputs
 */
#ifndef PTORACLE_H
#define PTORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── math (pitorch/ops/core/pt_math.c) ─────────────────────────────── */
float po_expf(float x);
float po_logf(float x);
float po_sinf(float x);
float po_cosf(float x);
float po_sqrtf(float x);

/* ── forward ops (pitorch/ops/core/pt_ops.c) ───────────────────────── */
void po_rmsnorm(float *o, const float *x, const float *w, int dim);
void po_softmax(float *x, int size);
void po_silu(float *x, int size);
void po_rope(float *q, float *k, int dim, int head_dim, int pos);
void po_vec_add(float *o, const float *a, const float *b, int size);
void po_vec_mul(float *o, const float *a, const float *b, int size);
void po_embedding_lookup(float *o, const float *table, int dim, int token);
int  po_argmax(const float *x, int n);
void po_smatvec(const float *W, const float *x, float *y, int out_dim, int in_dim);

/* ── GEMMs (pitorch/ops/gemm/gemm.c, gemm_rect.h, pt_train.c) ──────── */
void po_sgemm(const float *A, const float *B, float *C, int M, int K, int N);
void po_sgemm_rect(const float *A, const float *B, float *C,
                   int M, int K, int N, int accumulate);
void po_matmul_backward_input(float *d_x, const float *W, const float *d_y,
                              int out_dim, int in_dim);
void po_matmul_backward_weight(float *d_W, const float *d_y, const float *x,
                               int out_dim, int in_dim);
void po_matmul_backward_weight_batched(float *d_W, const float *d_y_all,
                                       const float *x_all, int out_dim,
                                       int in_dim, int T);

/* ── backward ops (pitorch/train/pt_backward_ops.c) ────────────────── */
void po_rmsnorm_backward(float *d_x, float *d_w, const float *d_o,
                         const float *x, const float *w, int dim);
void po_rope_backward(float *d_q, float *d_k, const float *d_q_out,
                      const float *d_k_out, int dim, int head_dim, int pos);
void po_softmax_backward(float *d_x, const float *d_y, const float *y, int size);
void po_silu_backward(float *d_x, const float *d_y, const float *x, int size);
void po_embedding_backward(float *d_table, const float *d_o, int dim, int token);

/* ── model (pitorch/model/llama2.c) ────────────────────────────────── */
typedef struct {
    int dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len;
} po_config_t;

/* Opaque model: weights point into a caller-owned llama2.c .bin blob. */
typedef struct po_model po_model_t;

void        po_load_config(po_config_t *cfg, const void *blob);
uint64_t    po_file_size(const void *blob);
po_model_t *po_model_new(void *blob, int max_T);
void        po_model_free(po_model_t *m);
void        po_reset_kv(po_model_t *m);
int         po_forward_step(po_model_t *m, int token);     /* pt.c:267-271 */
void        po_forward(po_model_t *m, int token, int pos);  /* llama2.c:201-206 */
const float *po_logits(const po_model_t *m);
const float *po_residual(const po_model_t *m);              /* s->x */
int         po_pos(const po_model_t *m);
/* Greedy generation over token ids (pt_text.c:314-379 with temperature 0
 * and the tokenizer replaced by ids).  Returns the number of entries
 * written to out (every forwarded position's next token). */
int         po_generate_greedy(po_model_t *m, const int *prompt, int n_prompt,
                               int max_tokens, int *out);

/* ── training (pitorch/train/pt_train.c, pitorch/pt.c:339-364) ─────── */
float po_forward_train(po_model_t *m, const int *tokens, int T);
void  po_backward(po_model_t *m, const int *tokens, int T);
void  po_sgd_update(po_model_t *m, float lr);
float po_train_step(po_model_t *m, const int *tokens, int T, float lr);
void  po_zero_grads(po_model_t *m);
/* Gradient buffer in pt_weights_t order (pt_train.c:342-370); tied wcls
 * aliases token_embedding.  n_params is written to *n. */
const float *po_grads(const po_model_t *m, int *n);
/* Training activations (read-only views for the parity tests). */
const float *po_train_logits(const po_model_t *m);       /* [T, V] */
const float *po_train_x_final(const po_model_t *m);      /* [T, D] */

#ifdef __cplusplus
}
#endif
#endif
