/*
 * llama2.c model files and seeded synthetic inputs.
 * Header and tensor order: pitorch/model/llama2.c:9-70.
 */
#include <math.h>
#include <string.h>

#include "pt.h"

/* llama2.c:9-19 */
void pt_load_config(pt_config_t *cfg, const void *data) {
    const int32_t *h = (const int32_t *)data;
    cfg->dim = h[0];
    cfg->hidden_dim = h[1];
    cfg->n_layers = h[2];
    cfg->n_heads = h[3];
    cfg->n_kv_heads = h[4];
    cfg->vocab_size = h[5] > 0 ? h[5] : -h[5];
    cfg->seq_len = h[6];
}

static uint64_t weight_floats(const pt_config_t *c, int shared) {
    uint64_t D = c->dim, H = c->hidden_dim, L = c->n_layers, V = c->vocab_size;
    uint64_t hd = D / c->n_heads, KV = (uint64_t)c->n_kv_heads * hd;
    uint64_t n = V * D + L * D + L * D * D + 2 * L * KV * D + L * D * D + L * D + 3 * L * H * D + D +
                 2 * ((uint64_t)c->seq_len * hd / 2);
    if (!shared) n += V * D;
    return n;
}

/* llama2.c:21-47, in 64-bit arithmetic. */
uint64_t pt_file_size(const void *data) {
    pt_config_t c;
    pt_load_config(&c, data);
    return 28 + 4 * weight_floats(&c, ((const int32_t *)data)[5] > 0);
}

uint64_t pt_synth_model_bytes(const pt_config_t *cfg) { return 28 + 4 * weight_floats(cfg, 1); }

/* splitmix64 (Steele, Lea, Flood 2014). */
static uint64_t sm64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in (0, 1]: 53 random bits */
static double unit(uint64_t *s) { return ((double)(sm64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0); }

static void fill_normal(uint64_t *s, float *p, uint64_t n, float std) {
    const double two_pi = 6.283185307179586476925286766559;
    uint64_t i = 0;
    while (i < n) {
        double r = sqrt(-2.0 * log(unit(s)));
        double a = two_pi * unit(s);
        p[i++] = (float)(std * r * cos(a));
        if (i < n) p[i++] = (float)(std * r * sin(a));
    }
}

int pt_synth_model(const pt_config_t *cfg, uint64_t seed, float std, void *out, uint64_t bytes) {
    if (!cfg || !out || cfg->dim <= 0 || cfg->n_heads <= 0 || cfg->dim % cfg->n_heads) return PTMI_ERR_ARG;
    if (bytes < pt_synth_model_bytes(cfg)) return PTMI_ERR_ARG;
    int32_t *h = (int32_t *)out;
    h[0] = cfg->dim; h[1] = cfg->hidden_dim; h[2] = cfg->n_layers; h[3] = cfg->n_heads;
    h[4] = cfg->n_kv_heads; h[5] = cfg->vocab_size; h[6] = cfg->seq_len;
    uint64_t D = cfg->dim, H = cfg->hidden_dim, L = cfg->n_layers, V = cfg->vocab_size;
    uint64_t hd = D / cfg->n_heads, KV = (uint64_t)cfg->n_kv_heads * hd;
    float *p = (float *)((char *)out + 28);
    uint64_t s = seed;
    /* file order: emb, rms_att, wq, wk, wv, wo, rms_ffn, w1, w2, w3,
     * rms_final, freq_cis_real, freq_cis_imag */
    fill_normal(&s, p, V * D, std);                 p += V * D;
    for (uint64_t i = 0; i < L * D; i++) p[i] = 1.0f;
    p += L * D;
    fill_normal(&s, p, L * D * D, std);             p += L * D * D;
    fill_normal(&s, p, 2 * L * KV * D, std);        p += 2 * L * KV * D;
    fill_normal(&s, p, L * D * D, std);             p += L * D * D;
    for (uint64_t i = 0; i < L * D; i++) p[i] = 1.0f;
    p += L * D;
    fill_normal(&s, p, 3 * L * H * D, std);         p += 3 * L * H * D;
    for (uint64_t i = 0; i < D; i++) p[i] = 1.0f;
    p += D;
    memset(p, 0, 2 * ((uint64_t)cfg->seq_len * hd / 2) * sizeof(float));
    return PTMI_OK;
}

void pt_seed_tokens(uint64_t seed, int n, int vocab, int *out) {
    uint64_t s = seed;
    for (int i = 0; i < n; i++) out[i] = (int)(sm64(&s) % (uint64_t)vocab);
}

void pt_seed_uniform(uint64_t seed, uint64_t n, float lo, float hi, float *out) {
    uint64_t s = seed;
    for (uint64_t i = 0; i < n; i++) out[i] = (float)(lo + (hi - lo) * ((double)(sm64(&s) >> 40) / 16777216.0));
}
