/*
 * pt.h — host API of the MI355X build, in C, with pitorch's call
 * signatures (pitorch/pt.h:23-104) so callers of pt_forward_step /
 * pt_train_step / the generate loop switch by changing the init call.
 *
 * The context owns a device-resident model in libptmi (include/ptmi.h):
 * decode steps are one hipGraph launch each, training steps run forward,
 * backward and SGD on the device.  ctx->matvec is ptmi_matvec, the
 * pt_matvec_fn drop-in, for callers that drive the layer code themselves
 * (pitorch/model/llama2.c pt_forward with the matvec pointer).
 *
 * Failures panic (message + abort), as the reference does with
 * demand()/panic(); the pt_try_* forms return a ptmi status instead.
 */
#ifndef PTAMD_PT_H
#define PTAMD_PT_H

#include <stddef.h>
#include <stdint.h>

#include "ptmi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* pitorch/model/llama2.h:10-18 */
typedef struct {
    int dim;
    int hidden_dim;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int vocab_size;
    int seq_len;
} pt_config_t;

/* pitorch/model/llama2.h:73-75 */
typedef void (*pt_matvec_fn)(const float *W, const float *x, float *y,
                             int out_dim, int in_dim);

/* ── trace (pitorch/profiler/trace.h:21-101): spans as Chrome-Tracing
 * JSON.  All functions are no-ops when t is NULL or t->enabled is 0.   */
#define PT_TRACE_MAX_EVENTS 4096
#define PT_TRACE_MAX_DEPTH  32

typedef struct {
    const char *name;
    const char *cat;       /* "fwd", "bwd", "train" */
    uint32_t    ts_us;     /* start (microseconds) */
    uint32_t    dur_us;    /* duration (microseconds) */
    int8_t      layer;     /* transformer layer, -1 = none */
    int8_t      depth;     /* nesting depth */
    uint32_t    hw_cycles; /* reference: V3D QPU cycles; 0 here */
    uint32_t    hw_stall;  /* reference: V3D TMU stall cycles; 0 here */
} pt_trace_event_t;

typedef struct {
    pt_trace_event_t events[PT_TRACE_MAX_EVENTS];
    int              count;
    int              enabled;
    struct {
        const char *name;
        const char *cat;
        uint32_t    ts_us;
        int8_t      layer;
    } stack[PT_TRACE_MAX_DEPTH];
    int              depth;
} pt_trace_t;

void     pt_trace_init(pt_trace_t *t);
void     pt_trace_begin(pt_trace_t *t, const char *name, const char *cat, int layer);
void     pt_trace_end(pt_trace_t *t);
void     pt_trace_reset(pt_trace_t *t);
uint32_t pt_time_us(void);
void     pt_trace_write_json(const pt_trace_t *t, const char *path);
void     pt_trace_write_meta(const char *path, const char *name, const char *model, int dim, int layers,
                             int vocab, const char *device, int num_qpus, int steps, float lr,
                             float final_loss, float total_time_s, const char *notes);
/* No reference counterpart: record an already finished span (the device
 * step's spans are added this way), and sizeof(pt_trace_t) for callers
 * that allocate it from another language.                              */
void     pt_trace_add(pt_trace_t *t, const char *name, const char *cat, int layer, int depth,
                      uint32_t ts_us, uint32_t dur_us);
size_t   pt_trace_size(void);

/* pitorch/pt.h:23-44, with the device model in place of host buffers. */
typedef struct {
    pt_config_t   cfg;
    int           shared_weights;
    pt_matvec_fn  matvec;        /* = ptmi_matvec */
    int           pos;           /* current decode position */
    int           max_T;         /* > 0: training buffers allocated */
    void         *weight_data;   /* caller's .bin blob (header + weights) */
    size_t        weight_bytes;
    ptmi_model_t *dev;
    float        *logits;        /* host copy, filled on demand */
    pt_trace_t   *trace;         /* pt_enable_trace; NULL = off */
    int           trace_owned;   /* allocated by pt_enable_trace */
} pt_context_t;

/* ── model file (pitorch/model/llama2.c:9-47) ── */
void     pt_load_config(pt_config_t *cfg, const void *data);
uint64_t pt_file_size(const void *data);

/* ── init / teardown: replaces pt_host_init / pt_pi_init (pt.c:38-114,
 * 232-248).  weight_data stays owned by the caller and must outlive ctx. */
int  pt_try_gpu_init(pt_context_t *ctx, void *weight_data, size_t bytes, int max_T);
void pt_gpu_init(pt_context_t *ctx, void *weight_data, size_t bytes, int max_T);
void pt_free(pt_context_t *ctx);

/* ── inference (pt.c:267-280) ── */
int  pt_forward_step(pt_context_t *ctx, int token);
int  pt_try_forward_step(pt_context_t *ctx, int token, int *next);
void pt_reset_kv(pt_context_t *ctx);
const float *pt_logits(pt_context_t *ctx);
void pt_print_config(const pt_context_t *ctx);

/* Greedy generation over token ids: the pt_generate loop
 * (pitorch/text/pt_text.c:314-361) at temperature 0, tokenizer excluded.
 * Writes the token chosen after each position to out; returns the number
 * of positions run (stops after a sampled BOS/EOS, pt_text.c:354).     */
int  pt_generate_ids(pt_context_t *ctx, const int *prompt, int n_prompt,
                     int max_tokens, int *out);

/* ── profiling (pt.c:322-335): with a trace enabled, pt_train_step runs
 * the device step without its graph and records the reference's span
 * tree (train_step, zero_grads, forward, embedding, layer, qkv,
 * attention, ffn, classifier, loss, backward, cls_transpose,
 * cls_weight_grad, transpose, wo, sgd; pt_train.c:171-866), plus
 * weight_grads (the layers' dW GEMMs in one launch), with HIP-event
 * times.  preallocated = NULL: the context allocates (and pt_free frees) it. */
void pt_enable_trace(pt_context_t *ctx, pt_trace_t *preallocated);
void pt_disable_trace(pt_context_t *ctx);

/* ── training (pt.c:339-364) ── */
float pt_train_step(pt_context_t *ctx, const int *tokens, int T, float lr);
int   pt_try_train_step(pt_context_t *ctx, const int *tokens, int T, float lr, float *loss);
/* Copy the trained device weights back into ctx->weight_data. */
int   pt_sync_weights(pt_context_t *ctx);

/* ── synthetic inputs (the benchmark configurations' model and ids) ──
 * A llama2.c .bin with weights ~ N(0, std) from splitmix64 + Box-Muller,
 * RMSNorm weights 1, freq_cis blocks 0, tied classifier (positive
 * vocab_size).  Deterministic for a given seed on every host.          */
uint64_t pt_synth_model_bytes(const pt_config_t *cfg);
int      pt_synth_model(const pt_config_t *cfg, uint64_t seed, float std,
                        void *out, uint64_t bytes);
/* n ids uniform in [0, vocab) from seed. */
void     pt_seed_tokens(uint64_t seed, int n, int vocab, int *out);
/* n floats uniform in [lo, hi) from seed (matvec sweep inputs). */
void     pt_seed_uniform(uint64_t seed, uint64_t n, float lo, float hi, float *out);

#ifdef __cplusplus
}
#endif
#endif
