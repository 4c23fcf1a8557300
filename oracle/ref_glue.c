/*
 * ref_glue.c — ctypes-friendly wrappers around the reference's own host
 * build (pitorch/pt.c context API), compiled against the reference headers
 * where they lie.  TEST INFRASTRUCTURE: linked only into oracle/_ref.
 *
 * ref_set_matvec() is the reference-side binding of the drop-in: it swaps
 * ctx->matvec (pitorch/pt.h:27) for any pt_matvec_fn, e.g. ptmi_matvec,
 * exactly as the reference's own tests swap smatvec_cpu in
 * (dev/tests/forward/test_forward.c:40-57).
 */
#include <stdlib.h>
#include "pt.h"
#include "pt_ops.h"

pt_context_t *ref_ctx_new(void *blob, int max_T) {
    pt_context_t *c = (pt_context_t *)calloc(1, sizeof(*c));
    pt_host_init(c, blob, max_T);
    return c;
}
void ref_ctx_free(pt_context_t *c) { pt_free(c); free(c); }
void ref_set_matvec(pt_context_t *c, pt_matvec_fn fn) { c->matvec = fn ? fn : smatvec_cpu; }
int ref_forward_step(pt_context_t *c, int token) { return pt_forward_step(c, token); }
void ref_reset_kv(pt_context_t *c) { pt_reset_kv(c); }
const float *ref_logits(pt_context_t *c) { return c->state.logits; }
float ref_train_step(pt_context_t *c, const int *tokens, int T, float lr) {
    return pt_train_step(c, tokens, T, lr);
}
const float *ref_grads(pt_context_t *c, int *n) { *n = c->grads._n_params; return c->grads._mem; }
const float *ref_train_logits(pt_context_t *c) { return c->acts.logits; }

/* pt_train_step, then `after(blob, bytes)`: the reference-side binding of
 * the drop-in for training.  pt_sgd_update (pitorch/train/pt_train.c:
 * 870-896) rewrites the host weights in place, so a caller whose
 * ctx->matvec serves resident device copies (ptmi_matvec) must re-upload
 * them after every step: after = ptmi_invalidate. */
typedef int (*ref_after_fn)(const void *, size_t);
float ref_train_step_then(pt_context_t *c, const int *tokens, int T, float lr, ref_after_fn after,
                          const void *blob, size_t bytes) {
    float loss = pt_train_step(c, tokens, T, lr);
    if (after) after(blob, bytes);
    return loss;
}

/* The reference's trace (pitorch/pt.c:322-335, profiler/trace.c). */
void ref_enable_trace(pt_context_t *c) { pt_enable_trace(c, NULL); }
pt_trace_t *ref_trace(pt_context_t *c) { return c->trace; }
size_t ref_trace_size(void) { return sizeof(pt_trace_t); }
