/*
 * pt_demo — a C caller of the pt.h API, in the shape of pitorch's
 * examples/generate.c:49-79 and examples/train.c:50-95: load a model,
 * initialise the context, then generate greedily or run SGD steps.  The
 * only change from the reference's callers is the init call
 * (pt_gpu_init in place of pt_pi_init / pt_host_init).  The model is the
 * seeded synthetic .bin the benchmark configurations use (no checkpoint
 * or tokenizer is available), and tokens are ids.
 *
 *   pt_demo generate D H L NH NKV V S MODEL_SEED PROMPT_SEED N_PROMPT MAX_TOKENS
 *       prints "prompt: ..." and the chosen ids twice: from pt_generate_ids
 *       and from a pt_forward_step loop with prompt forcing
 *   pt_demo train D H L NH NKV V S MODEL_SEED TRAIN_SEED T LR STEPS [TRACE_DIR]
 *       prints "loss <step> <value>" per pt_train_step; with TRACE_DIR the
 *       steps run traced (pt_enable_trace, as the reference's
 *       dev/host/test_train_profiled.c:44-104) and TRACE_DIR/trace.json and
 *       TRACE_DIR/meta.json are written
 *
 * Exit status 0 on success; failures abort with a message, as the
 * reference's panic() does.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "pt.h"

static void usage(void) {
    fprintf(stderr,
            "usage: pt_demo generate D H L NH NKV V S MODEL_SEED PROMPT_SEED N_PROMPT MAX_TOKENS\n"
            "       pt_demo train    D H L NH NKV V S MODEL_SEED TRAIN_SEED T LR STEPS [TRACE_DIR]\n");
    exit(2);
}

static void *synth(const pt_config_t *cfg, unsigned long long seed, size_t *bytes) {
    *bytes = (size_t)pt_synth_model_bytes(cfg);
    void *blob = malloc(*bytes);
    if (!blob || pt_synth_model(cfg, seed, 0.02f, blob, *bytes) != 0) {
        fprintf(stderr, "pt_demo: cannot build the synthetic model\n");
        exit(1);
    }
    return blob;
}

static int generate(const pt_config_t *cfg, unsigned long long mseed, unsigned long long pseed, int n_prompt,
                    int max_tokens) {
    size_t bytes;
    void *blob = synth(cfg, mseed, &bytes);
    pt_context_t ctx;
    pt_gpu_init(&ctx, blob, bytes, 0);
    pt_print_config(&ctx);

    int *prompt = malloc(sizeof(int) * (size_t)n_prompt);
    int *out = malloc(sizeof(int) * (size_t)(max_tokens + 1));
    pt_seed_tokens(pseed, n_prompt, cfg->vocab_size, prompt);
    printf("prompt:");
    for (int i = 0; i < n_prompt; i++) printf(" %d", prompt[i]);
    printf("\n");

    /* the pt_generate loop (pt_text.c:314-361) at temperature 0 */
    int n = pt_generate_ids(&ctx, prompt, n_prompt, max_tokens, out);
    printf("generate:");
    for (int i = 0; i < n; i++) printf(" %d", out[i]);
    printf("\n");

    /* the same loop written against pt_forward_step (pt.c:267-271) */
    if (max_tokens > cfg->seq_len) max_tokens = cfg->seq_len;
    pt_reset_kv(&ctx);
    printf("forward_step:");
    int token = prompt[0];
    for (int pos = 0; pos < max_tokens; pos++) {
        int next = pt_forward_step(&ctx, token);
        if (pos + 1 < n_prompt) next = prompt[pos + 1];
        printf(" %d", next);
        if (pos + 1 >= n_prompt && (next == 1 || next == 2)) break;
        token = next;
    }
    printf("\n");
    pt_free(&ctx);
    free(prompt);
    free(out);
    free(blob);
    return 0;
}

static int train(const pt_config_t *cfg, unsigned long long mseed, unsigned long long tseed, int T, float lr,
                 int steps, const char *trace_dir) {
    size_t bytes;
    void *blob = synth(cfg, mseed, &bytes);
    pt_context_t ctx;
    pt_gpu_init(&ctx, blob, bytes, T);
    if (trace_dir) pt_enable_trace(&ctx, NULL);
    int *tokens = malloc(sizeof(int) * (size_t)T);
    pt_seed_tokens(tseed, T, cfg->vocab_size, tokens);
    const uint32_t t0 = pt_time_us();
    float loss = 0.0f;
    for (int s = 0; s < steps; s++) {
        loss = pt_train_step(&ctx, tokens, T, lr);
        printf("loss %d %.6f\n", s, loss);
    }
    if (trace_dir) {
        char path[1024];
        mkdir(trace_dir, 0755);                 /* as dev/host/test_train_profiled.c:88 */
        snprintf(path, sizeof path, "%s/trace.json", trace_dir);
        pt_trace_write_json(ctx.trace, path);
        FILE *check = fopen(path, "r");
        if (!check) {
            fprintf(stderr, "pt_demo: could not write %s\n", path);
            return 1;
        }
        fclose(check);
        printf("trace %s %d events\n", path, ctx.trace->count);
        snprintf(path, sizeof path, "%s/meta.json", trace_dir);
        pt_trace_write_meta(path, "synthetic training, traced", "synthetic", cfg->dim, cfg->n_layers,
                            cfg->vocab_size, "mi355x", 0, steps, lr, loss, (float)(pt_time_us() - t0) * 1e-6f,
                            "device spans timed with HIP events");
    }
    if (pt_sync_weights(&ctx) != 0) {
        fprintf(stderr, "pt_demo: pt_sync_weights: %s\n", ptmi_last_error());
        return 1;
    }
    pt_free(&ctx);
    free(tokens);
    free(blob);
    return 0;
}

int main(int argc, char **argv) {
    if (argc < 2) usage();
    const int gen = !strcmp(argv[1], "generate"), trn = !strcmp(argv[1], "train");
    if (!(gen && argc == 13) && !(trn && (argc == 14 || argc == 15))) usage();
    pt_config_t cfg;
    int *f = &cfg.dim;
    for (int i = 0; i < 7; i++) f[i] = atoi(argv[2 + i]);
    const unsigned long long mseed = strtoull(argv[9], NULL, 10), seed2 = strtoull(argv[10], NULL, 10);
    if (gen) return generate(&cfg, mseed, seed2, atoi(argv[11]), atoi(argv[12]));
    return train(&cfg, mseed, seed2, atoi(argv[11]), (float)atof(argv[12]), atoi(argv[13]), argc == 15 ? argv[14] : NULL);
}
