/*
 * pt_host.c — pitorch's context API (pitorch/pt.c) over libptmi.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pt.h"

static void panic_status(const char *what, int st) {
    fprintf(stderr, "%s failed (status %d): %s\n", what, st, ptmi_last_error());
    abort();
}

int pt_try_gpu_init(pt_context_t *ctx, void *weight_data, size_t bytes, int max_T) {
    memset(ctx, 0, sizeof(*ctx));
    if (!weight_data || bytes < 28) return PTMI_ERR_ARG;
    pt_load_config(&ctx->cfg, weight_data);
    ctx->shared_weights = ((const int32_t *)weight_data)[5] > 0;
    ctx->matvec = ptmi_matvec;
    ctx->max_T = max_T;
    ctx->weight_data = weight_data;
    ctx->weight_bytes = bytes;
    int st = ptmi_model_create(weight_data, bytes, max_T, &ctx->dev);
    if (st) return st;
    ctx->logits = (float *)malloc((size_t)ctx->cfg.vocab_size * sizeof(float));
    if (!ctx->logits) {
        ptmi_model_destroy(ctx->dev);
        ctx->dev = NULL;
        return PTMI_ERR_OOM;
    }
    return PTMI_OK;
}

void pt_gpu_init(pt_context_t *ctx, void *weight_data, size_t bytes, int max_T) {
    int st = pt_try_gpu_init(ctx, weight_data, bytes, max_T);
    if (st) panic_status("pt_gpu_init", st);
}

void pt_free(pt_context_t *ctx) {
    /* the model's hold on the blob's device copy ends with it */
    if (ctx->dev) ptmi_model_destroy(ctx->dev);
    ctx->dev = NULL;
    free(ctx->logits);
    ctx->logits = NULL;
    if (ctx->trace_owned) free(ctx->trace);
    ctx->trace = NULL;
    ctx->trace_owned = 0;
}

/* pt.c:267-271: forward `token` at ctx->pos, pos++, greedy next token. */
int pt_try_forward_step(pt_context_t *ctx, int token, int *next) {
    int st = ptmi_model_forward_step(ctx->dev, token, next);
    if (st == PTMI_OK) ctx->pos++;
    return st;
}

int pt_forward_step(pt_context_t *ctx, int token) {
    int next = 0;
    int st = pt_try_forward_step(ctx, token, &next);
    if (st) panic_status("pt_forward_step", st);
    return next;
}

/* pt.c:273-280 */
void pt_reset_kv(pt_context_t *ctx) {
    int st = ptmi_model_reset_kv(ctx->dev);
    if (st) panic_status("pt_reset_kv", st);
    ctx->pos = 0;
}

const float *pt_logits(pt_context_t *ctx) {
    int st = ptmi_model_logits(ctx->dev, ctx->logits);
    if (st) panic_status("pt_logits", st);
    return ctx->logits;
}

/* pt.c:282-301 (host branch) */
void pt_print_config(const pt_context_t *ctx) {
    const pt_config_t *c = &ctx->cfg;
    printf("pitorch (%dd %dL %dKv) | MI355X\n", c->dim, c->n_layers, c->vocab_size / 1000);
    printf("  dim=%d hidden=%d L=%d H=%d kv=%d V=%d seq=%d\n", c->dim, c->hidden_dim, c->n_layers,
           c->n_heads, c->n_kv_heads, c->vocab_size, c->seq_len);
    if (ctx->max_T > 0) printf("  training: max_T=%d\n", ctx->max_T);
}

int pt_generate_ids(pt_context_t *ctx, const int *prompt, int n_prompt, int max_tokens, int *out) {
    int n = 0;
    int st = ptmi_model_generate(ctx->dev, prompt, n_prompt, max_tokens, 1, out, &n);
    if (st) panic_status("pt_generate_ids", st);
    ctx->pos = ptmi_model_pos(ctx->dev);
    return n;
}

/* pt.c:322-335 */
void pt_enable_trace(pt_context_t *ctx, pt_trace_t *preallocated) {
    if (preallocated) {
        if (ctx->trace_owned) free(ctx->trace);
        ctx->trace = preallocated;
        ctx->trace_owned = 0;
    } else if (!ctx->trace) {
        ctx->trace = (pt_trace_t *)malloc(sizeof(pt_trace_t));
        ctx->trace_owned = ctx->trace != NULL;
    }
    if (ctx->trace) pt_trace_init(ctx->trace);
}

void pt_disable_trace(pt_context_t *ctx) {
    if (ctx->trace) ctx->trace->enabled = 0;
}

/* pt.c:339-364.  Traced: the device step's spans, placed on the host clock
 * at the call, in the order the device step ends them. */
int pt_try_train_step(pt_context_t *ctx, const int *tokens, int T, float lr, float *loss) {
    pt_trace_t *tr = ctx->trace;
    if (!tr || !tr->enabled) return ptmi_model_train_step(ctx->dev, tokens, T, lr, loss);
    ptmi_span_t *spans = (ptmi_span_t *)malloc(sizeof(ptmi_span_t) * PT_TRACE_MAX_EVENTS);
    if (!spans) return ptmi_model_train_step(ctx->dev, tokens, T, lr, loss);
    int n = 0;
    const uint32_t t0 = pt_time_us();
    const int st = ptmi_model_train_step_trace(ctx->dev, tokens, T, lr, loss, spans, PT_TRACE_MAX_EVENTS, &n);
    if (st == 0) {
        for (int i = 0; i < n; i++)
            pt_trace_add(tr, spans[i].name, spans[i].cat, spans[i].layer, tr->depth + spans[i].depth,
                         t0 + (uint32_t)(spans[i].start_us + 0.5), (uint32_t)(spans[i].dur_us + 0.5));
    }
    free(spans);
    return st;
}

float pt_train_step(pt_context_t *ctx, const int *tokens, int T, float lr) {
    float loss = 0.0f;
    int st = pt_try_train_step(ctx, tokens, T, lr, &loss);
    if (st) panic_status("pt_train_step", st);
    return loss;
}

int pt_sync_weights(pt_context_t *ctx) {
    return ptmi_model_read_weights(ctx->dev, ctx->weight_data, ctx->weight_bytes);
}
