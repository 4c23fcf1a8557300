/*
 * ptoracle.c — CPU restatement of the reference algorithms (test oracle).
 * See ptoracle.h for scope and pinning.  Build with -O2 -ffp-contract=off:
 * every expression below is evaluated in the same order, with the same
 * float literals and conversions, as the cited reference line, and without
 * fused multiply-adds, so results match the reference bit for bit.
 */
#include "ptoracle.h"

#include <stdlib.h>
#include <string.h>

/* ═══ math — pitorch/ops/core/pt_math.c ══════════════════════════════ */

static inline float bits_to_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* pt_math.c:8-25: n = round-half-away(x/ln2), r = x - n*ln2, degree-5
 * Horner polynomial for e^r, times 2^n assembled in the exponent field. */
float po_expf(float x) {
    if (x > 88.7f) return 3.4028235e+38f;
    if (x < -87.3f) return 0.0f;
    const float ln2 = 0.6931471805599453f, inv_ln2 = 1.4426950408889634f;
    float t = x * inv_ln2;
    int n = (int)(t + (t >= 0 ? 0.5f : -0.5f));
    float r = x - (float)n * ln2;
    float poly = 0.0416666667f + r * 0.0083333333f;
    poly = 0.1666666667f + r * poly;
    poly = 0.5f + r * poly;
    poly = 1.0f + r * poly;
    poly = 1.0f + r * poly;
    return poly * bits_to_f((uint32_t)(n + 127) << 23);
}

/* pt_math.c:31-44: x = m*2^e, m folded into (0.707, 1.414], 9-term
 * series for ln(1+f), plus e*ln2. */
float po_logf(float x) {
    if (x <= 0.0f) return -3.4028235e+38f;
    uint32_t u = f_to_bits(x);
    int e = (int)((u >> 23) & 0xFF) - 127;
    float m = bits_to_f((u & 0x007FFFFFu) | 0x3F800000u);
    if (m > 1.41421356f) { m *= 0.5f; e++; }
    float f = m - 1.0f;
    float s = -0.125f + f * 0.11111111f;
    s = 0.14285714f + f * s;
    s = -0.16666667f + f * s;
    s = 0.2f + f * s;
    s = -0.25f + f * s;
    s = 0.33333333f + f * s;
    s = -0.5f + f * s;
    s = 1.0f + f * s;
    return f * s + (float)e * 0.69314718f;
}

/* pt_math.c:52-62: reduce to [-pi, pi] by rounding x/(2pi). */
static float wrap_pi(float x) {
    float k = x * 0.15915494309190f;
    k = (float)(int)(k + (k >= 0 ? 0.5f : -0.5f));
    return x - k * 6.28318530717959f;
}

/* pt_math.c:64-74: fold into [-pi/2, pi/2] with sin(pi-x)=sin(x), odd
 * degree-9 polynomial. */
float po_sinf(float x) {
    const float pi = 3.14159265358979f, half_pi = 1.57079632679490f;
    x = wrap_pi(x);
    if (x > half_pi) x = pi - x;
    else if (x < -half_pi) x = -pi - x;
    float z = x * x;
    float s = -0.00019841270f + z * 0.00000275573f;
    s = 0.00833333333f + z * s;
    s = -0.16666666667f + z * s;
    s = 1.0f + z * s;
    return x * s;
}

/* pt_math.c:76-87: as sin, with the sign flip cos(pi-x) = -cos(x). */
float po_cosf(float x) {
    const float pi = 3.14159265358979f, half_pi = 1.57079632679490f;
    x = wrap_pi(x);
    float sign = 1.0f;
    if (x > half_pi) { x = pi - x; sign = -1.0f; }
    else if (x < -half_pi) { x = -pi - x; sign = -1.0f; }
    float z = x * x;
    float c = -0.00138888889f + z * 0.00002480159f;
    c = 0.04166666667f + z * c;
    c = -0.50000000000f + z * c;
    c = 1.0f + z * c;
    return sign * c;
}

/* pt_math.c:92-102: exponent-halving seed, three Newton steps. */
float po_sqrtf(float x) {
    if (x <= 0.0f) return 0.0f;
    float y = bits_to_f(0x1fbd1df5u + (f_to_bits(x) >> 1));
    for (int it = 0; it < 3; it++) y = 0.5f * (y + x / y);
    return y;
}

/* ═══ forward ops — pitorch/ops/core/pt_ops.c ════════════════════════ */

/* pt_ops.c:5-12 */
void po_rmsnorm(float *o, const float *x, const float *w, int dim) {
    float ss = 0.0f;
    for (int i = 0; i < dim; i++) ss += x[i] * x[i];
    float inv = 1.0f / po_sqrtf(ss / dim + 1e-5f);
    for (int i = 0; i < dim; i++) o[i] = x[i] * inv * w[i];
}

/* pt_ops.c:14-26 */
void po_softmax(float *x, int size) {
    float mx = x[0];
    for (int i = 1; i < size; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < size; i++) { x[i] = po_expf(x[i] - mx); sum += x[i]; }
    float inv = 1.0f / sum;
    for (int i = 0; i < size; i++) x[i] *= inv;
}

/* pt_ops.c:28-31 */
void po_silu(float *x, int size) {
    for (int i = 0; i < size; i++) x[i] = x[i] / (1.0f + po_expf(-x[i]));
}

/* pt_ops.c:33-49: frequency exp(-ln(1e4) * (i mod hd) / hd), q and k
 * rotated over the same `dim` pairs. */
static void rope_angle(int i, int head_dim, int pos, float *c, float *s) {
    int hi = i % head_dim;
    float freq = po_expf(-9.210340372f * (float)hi / (float)head_dim);
    float ang = (float)pos * freq;
    *c = po_cosf(ang);
    *s = po_sinf(ang);
}

void po_rope(float *q, float *k, int dim, int head_dim, int pos) {
    for (int i = 0; i < dim; i += 2) {
        float c, s;
        rope_angle(i, head_dim, pos, &c, &s);
        float a = q[i], b = q[i + 1];
        q[i] = a * c - b * s;
        q[i + 1] = a * s + b * c;
        a = k[i]; b = k[i + 1];
        k[i] = a * c - b * s;
        k[i + 1] = a * s + b * c;
    }
}

/* pt_ops.c:51-59 */
void po_vec_add(float *o, const float *a, const float *b, int size) {
    for (int i = 0; i < size; i++) o[i] = a[i] + b[i];
}
void po_vec_mul(float *o, const float *a, const float *b, int size) {
    for (int i = 0; i < size; i++) o[i] = a[i] * b[i];
}

/* pt_ops.c:61-63 */
void po_embedding_lookup(float *o, const float *table, int dim, int token) {
    memcpy(o, table + (size_t)token * dim, (size_t)dim * sizeof(float));
}

/* pt_ops.c:65-70: first index of the maximum (strict >). */
int po_argmax(const float *x, int n) {
    int best = 0;
    for (int i = 1; i < n; i++) if (x[i] > x[best]) best = i;
    return best;
}

/* pt_ops.c:72-80: y[i] = sum_j W[i][j]*x[j], one dependent fp32 add
 * chain per row in j order, starting from +0.0f. */
void po_smatvec(const float *W, const float *x, float *y, int out_dim, int in_dim) {
    for (int i = 0; i < out_dim; i++) {
        const float *row = W + (size_t)i * in_dim;
        float acc = 0.0f;
        for (int j = 0; j < in_dim; j++) acc += row[j] * x[j];
        y[i] = acc;
    }
}

/* ═══ GEMMs ══════════════════════════════════════════════════════════ */

/* pitorch/ops/gemm/gemm.c:14-23: C = A.B, k-ordered per element. */
void po_sgemm(const float *A, const float *B, float *C, int M, int K, int N) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc += A[(size_t)i * K + k] * B[(size_t)k * N + j];
            C[(size_t)i * N + j] = acc;
        }
}

/* pitorch/ops/gemm/gemm_rect.h:12-26 semantics: C (+)= A[M,K].B[K,N].
 * The reference QPU kernel's order is not observable from the host; the
 * oracle uses sgemm_cpu's k order and adds the existing C last. */
void po_sgemm_rect(const float *A, const float *B, float *C,
                   int M, int K, int N, int accumulate) {
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc += A[(size_t)i * K + k] * B[(size_t)k * N + j];
            size_t o = (size_t)i * N + j;
            C[o] = accumulate ? C[o] + acc : acc;
        }
}

/* pitorch/train/pt_backward_ops.c:32-41: d_x[j] += sum_i W[i][j]*d_y[i]. */
void po_matmul_backward_input(float *d_x, const float *W, const float *d_y,
                              int out_dim, int in_dim) {
    for (int j = 0; j < in_dim; j++) {
        float acc = 0.0f;
        for (int i = 0; i < out_dim; i++) acc += W[(size_t)i * in_dim + j] * d_y[i];
        d_x[j] += acc;
    }
}

/* pitorch/train/pt_backward_ops.c:43-49: rank-1 update. */
void po_matmul_backward_weight(float *d_W, const float *d_y, const float *x,
                               int out_dim, int in_dim) {
    for (int i = 0; i < out_dim; i++)
        for (int j = 0; j < in_dim; j++)
            d_W[(size_t)i * in_dim + j] += d_y[i] * x[j];
}

/* pitorch/train/pt_train.c:475-492: d_W[i][j] += dY[t][i]*X[t][j] for
 * t = 0..T-1 in order.  The reference tiles i for cache reuse only; each
 * element still sees its T products in t order, as here. */
void po_matmul_backward_weight_batched(float *d_W, const float *d_y_all,
                                       const float *x_all, int out_dim,
                                       int in_dim, int T) {
    for (int i = 0; i < out_dim; i++) {
        float *dw = d_W + (size_t)i * in_dim;
        for (int t = 0; t < T; t++) {
            float g = d_y_all[(size_t)t * out_dim + i];
            const float *x = x_all + (size_t)t * in_dim;
            for (int j = 0; j < in_dim; j++) dw[j] += g * x[j];
        }
    }
}

/* ═══ backward ops — pitorch/train/pt_backward_ops.c ═════════════════ */

/* :4-30 */
void po_rmsnorm_backward(float *d_x, float *d_w, const float *d_o,
                         const float *x, const float *w, int dim) {
    float ss = 0.0f;
    for (int i = 0; i < dim; i++) ss += x[i] * x[i];
    ss = ss / dim + 1e-5f;
    float inv = 1.0f / po_sqrtf(ss);
    for (int i = 0; i < dim; i++) d_w[i] += d_o[i] * x[i] * inv;
    float dot = 0.0f;
    for (int i = 0; i < dim; i++) dot += d_o[i] * w[i] * x[i];
    float coeff = inv * inv * inv / (float)dim;
    for (int i = 0; i < dim; i++) d_x[i] += inv * d_o[i] * w[i] - coeff * dot * x[i];
}

/* :52-69: inverse rotation by the forward angle. */
void po_rope_backward(float *d_q, float *d_k, const float *d_q_out,
                      const float *d_k_out, int dim, int head_dim, int pos) {
    for (int i = 0; i < dim; i += 2) {
        float c, s;
        rope_angle(i, head_dim, pos, &c, &s);
        d_q[i] += d_q_out[i] * c + d_q_out[i + 1] * s;
        d_q[i + 1] += -d_q_out[i] * s + d_q_out[i + 1] * c;
        d_k[i] += d_k_out[i] * c + d_k_out[i + 1] * s;
        d_k[i + 1] += -d_k_out[i] * s + d_k_out[i + 1] * c;
    }
}

/* :71-79 */
void po_softmax_backward(float *d_x, const float *d_y, const float *y, int size) {
    float dot = 0.0f;
    for (int i = 0; i < size; i++) dot += d_y[i] * y[i];
    for (int i = 0; i < size; i++) d_x[i] += y[i] * (d_y[i] - dot);
}

/* :81-88 */
void po_silu_backward(float *d_x, const float *d_y, const float *x, int size) {
    for (int i = 0; i < size; i++) {
        float sig = 1.0f / (1.0f + po_expf(-x[i]));
        d_x[i] += d_y[i] * sig * (1.0f + x[i] * (1.0f - sig));
    }
}

/* :90-95 */
void po_embedding_backward(float *d_table, const float *d_o, int dim, int token) {
    for (int i = 0; i < dim; i++) d_table[(size_t)token * dim + i] += d_o[i];
}

/* ═══ model — pitorch/model/llama2.c ═════════════════════════════════ */

typedef struct {
    float *emb, *rms_att, *wq, *wk, *wv, *wo, *rms_ffn, *w1, *w2, *w3,
          *rms_final, *wcls;
} po_weights_t;

struct po_model {
    po_config_t c;
    int shared, kv_dim, head_dim;
    po_weights_t w;
    /* decode state (llama2.h:35-48) */
    float *x, *xb, *xb2, *q, *k, *v, *hb, *hb2, *att, *logits, *kc, *vc;
    int pos;
    /* training (pt_train.h:34-50, 76-86, 103-129) */
    int max_T;
    float *res, *res_att, *xb_att, *aq, *ak, *av, *aatt, *att_out, *xb_ffn,
          *ahb, *ahb2, *x_final, *tlogits, *scratch;
    float *gmem; int n_params; po_weights_t g;
    float *d_res, *d_aout, *d_q, *d_k, *d_v, *d_xb, *d_qpre, *d_kpre,
          *d_hid, *d_hid2, *d_att_s, *d_pre_sm, *d_logit_all, *drt_wo_all,
          *d_qpre_all, *d_kpre_all, *sh_all, *d_hid_all, *d_hid2_all,
          *drt_ffn_all, *d_temp;
};

/* llama2.c:9-19 */
void po_load_config(po_config_t *cfg, const void *blob) {
    const int32_t *h = (const int32_t *)blob;
    cfg->dim = h[0]; cfg->hidden_dim = h[1]; cfg->n_layers = h[2];
    cfg->n_heads = h[3]; cfg->n_kv_heads = h[4];
    cfg->vocab_size = h[5] > 0 ? h[5] : -h[5];
    cfg->seq_len = h[6];
}

/* llama2.c:21-47 (64-bit here; the reference sums in 32-bit unsigned). */
uint64_t po_file_size(const void *blob) {
    po_config_t c; po_load_config(&c, blob);
    int shared = ((const int32_t *)blob)[5] > 0;
    uint64_t hd = (uint64_t)(c.dim / c.n_heads), kv = (uint64_t)c.n_kv_heads * hd;
    uint64_t D = c.dim, H = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
    uint64_t n = V * D + L * D + L * D * D + 2 * L * kv * D + L * D * D + L * D
               + 3 * L * H * D + D + 2 * ((uint64_t)c.seq_len * hd / 2);
    if (!shared) n += V * D;
    return 28 + 4 * n;
}

/* llama2.c:49-70: tensors in file order after the 28-byte header; the two
 * freq_cis blocks are skipped; positive vocab_size means wcls is tied. */
static void load_weights(po_model_t *m, void *blob) {
    const po_config_t *c = &m->c;
    float *p = (float *)((char *)blob + 28);
    size_t D = c->dim, H = c->hidden_dim, L = c->n_layers, KV = m->kv_dim;
    m->w.emb = p;       p += (size_t)c->vocab_size * D;
    m->w.rms_att = p;   p += L * D;
    m->w.wq = p;        p += L * D * D;
    m->w.wk = p;        p += L * KV * D;
    m->w.wv = p;        p += L * KV * D;
    m->w.wo = p;        p += L * D * D;
    m->w.rms_ffn = p;   p += L * D;
    m->w.w1 = p;        p += L * H * D;
    m->w.w2 = p;        p += L * D * H;
    m->w.w3 = p;        p += L * H * D;
    m->w.rms_final = p; p += D;
    p += (size_t)c->seq_len * m->head_dim / 2;
    p += (size_t)c->seq_len * m->head_dim / 2;
    m->w.wcls = m->shared ? m->w.emb : p;
}

static float *zalloc(size_t n) { return (float *)calloc(n ? n : 1, sizeof(float)); }

po_model_t *po_model_new(void *blob, int max_T) {
    po_model_t *m = (po_model_t *)calloc(1, sizeof(*m));
    po_load_config(&m->c, blob);
    m->shared = ((const int32_t *)blob)[5] > 0;
    m->head_dim = m->c.dim / m->c.n_heads;
    m->kv_dim = m->c.n_kv_heads * m->head_dim;
    load_weights(m, blob);
    size_t D = m->c.dim, H = m->c.hidden_dim, L = m->c.n_layers, KV = m->kv_dim;
    size_t V = m->c.vocab_size, S = m->c.seq_len, NH = m->c.n_heads;
    m->x = zalloc(D); m->xb = zalloc(D); m->xb2 = zalloc(D); m->q = zalloc(D);
    m->k = zalloc(KV); m->v = zalloc(KV); m->hb = zalloc(H); m->hb2 = zalloc(H);
    m->att = zalloc(NH * S); m->logits = zalloc(V);
    m->kc = zalloc(L * S * KV); m->vc = zalloc(L * S * KV);
    m->max_T = max_T;
    if (max_T > 0) {
        size_t T = max_T;
        m->res = zalloc((L + 1) * T * D); m->res_att = zalloc(L * T * D);
        m->xb_att = zalloc(L * T * D); m->aq = zalloc(L * T * D);
        m->ak = zalloc(L * T * KV); m->av = zalloc(L * T * KV);
        m->aatt = zalloc(L * NH * T * T); m->att_out = zalloc(L * T * D);
        m->xb_ffn = zalloc(L * T * D); m->ahb = zalloc(L * T * H);
        m->ahb2 = zalloc(L * T * H); m->x_final = zalloc(T * D);
        m->tlogits = zalloc(T * V); m->scratch = zalloc(H > D ? H : D);
        /* pt_train.c:342-370 */
        size_t n = V * D + L * D + L * D * D + 2 * L * KV * D + L * D * D + L * D
                 + 3 * L * H * D + D + (m->shared ? 0 : V * D);
        m->gmem = zalloc(n); m->n_params = (int)n;
        float *p = m->gmem;
        m->g.emb = p; p += V * D;       m->g.rms_att = p; p += L * D;
        m->g.wq = p; p += L * D * D;    m->g.wk = p; p += L * KV * D;
        m->g.wv = p; p += L * KV * D;   m->g.wo = p; p += L * D * D;
        m->g.rms_ffn = p; p += L * D;   m->g.w1 = p; p += L * H * D;
        m->g.w2 = p; p += L * D * H;    m->g.w3 = p; p += L * H * D;
        m->g.rms_final = p; p += D;
        m->g.wcls = m->shared ? m->g.emb : p;
        m->d_res = zalloc(T * D); m->d_aout = zalloc(T * D); m->d_q = zalloc(T * D);
        m->d_k = zalloc(T * KV); m->d_v = zalloc(T * KV); m->d_xb = zalloc(D);
        m->d_qpre = zalloc(D); m->d_kpre = zalloc(KV); m->d_hid = zalloc(H);
        m->d_hid2 = zalloc(H); m->d_att_s = zalloc(T); m->d_pre_sm = zalloc(T);
        m->d_logit_all = zalloc(T * V); m->drt_wo_all = zalloc(T * D);
        m->d_qpre_all = zalloc(T * D); m->d_kpre_all = zalloc(T * KV);
        m->sh_all = zalloc(T * H); m->d_hid_all = zalloc(T * H);
        m->d_hid2_all = zalloc(T * H); m->drt_ffn_all = zalloc(T * D);
        m->d_temp = zalloc(H > D ? H : D);
    }
    return m;
}

void po_model_free(po_model_t *m) {
    if (!m) return;
    float *bufs[] = {m->x, m->xb, m->xb2, m->q, m->k, m->v, m->hb, m->hb2, m->att,
                     m->logits, m->kc, m->vc, m->res, m->res_att, m->xb_att, m->aq,
                     m->ak, m->av, m->aatt, m->att_out, m->xb_ffn, m->ahb, m->ahb2,
                     m->x_final, m->tlogits, m->scratch, m->gmem, m->d_res, m->d_aout,
                     m->d_q, m->d_k, m->d_v, m->d_xb, m->d_qpre, m->d_kpre, m->d_hid,
                     m->d_hid2, m->d_att_s, m->d_pre_sm, m->d_logit_all, m->drt_wo_all,
                     m->d_qpre_all, m->d_kpre_all, m->sh_all, m->d_hid_all,
                     m->d_hid2_all, m->drt_ffn_all, m->d_temp};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++) free(bufs[i]);
    free(m);
}

/* pt.c:273-280 */
void po_reset_kv(po_model_t *m) {
    size_t n = (size_t)m->c.n_layers * m->c.seq_len * m->kv_dim;
    memset(m->kc, 0, n * sizeof(float));
    memset(m->vc, 0, n * sizeof(float));
    m->pos = 0;
}

/* llama2.c:127-192: one token through layers [0, L). */
static void forward_layers(po_model_t *m, int pos) {
    const po_config_t *c = &m->c;
    int D = c->dim, H = c->hidden_dim, hd = m->head_dim, KV = m->kv_dim;
    int kv_mul = c->n_heads / c->n_kv_heads;
    float scale = 1.0f / po_sqrtf((float)hd);
    for (int l = 0; l < c->n_layers; l++) {
        po_rmsnorm(m->xb, m->x, m->w.rms_att + (size_t)l * D, D);
        po_smatvec(m->w.wq + (size_t)l * D * D, m->xb, m->q, D, D);
        po_smatvec(m->w.wk + (size_t)l * KV * D, m->xb, m->k, KV, D);
        po_smatvec(m->w.wv + (size_t)l * KV * D, m->xb, m->v, KV, D);
        po_rope(m->q, m->k, D, hd, pos);
        size_t lo = (size_t)l * c->seq_len * KV;
        memcpy(m->kc + lo + (size_t)pos * KV, m->k, KV * sizeof(float));
        memcpy(m->vc + lo + (size_t)pos * KV, m->v, KV * sizeof(float));
        for (int h = 0; h < c->n_heads; h++) {
            const float *qh = m->q + h * hd;
            float *ah = m->att + (size_t)h * c->seq_len;
            size_t ko = (size_t)(h / kv_mul) * hd;
            for (int t = 0; t <= pos; t++) {
                const float *kt = m->kc + lo + (size_t)t * KV + ko;
                float s = 0.0f;
                for (int i = 0; i < hd; i++) s += qh[i] * kt[i];
                ah[t] = s * scale;
            }
            po_softmax(ah, pos + 1);
            float *oh = m->xb + h * hd;
            memset(oh, 0, hd * sizeof(float));
            for (int t = 0; t <= pos; t++) {
                const float *vt = m->vc + lo + (size_t)t * KV + ko;
                float a = ah[t];
                for (int i = 0; i < hd; i++) oh[i] += a * vt[i];
            }
        }
        po_smatvec(m->w.wo + (size_t)l * D * D, m->xb, m->xb2, D, D);
        po_vec_add(m->x, m->x, m->xb2, D);
        po_rmsnorm(m->xb, m->x, m->w.rms_ffn + (size_t)l * D, D);
        po_smatvec(m->w.w1 + (size_t)l * H * D, m->xb, m->hb, H, D);
        po_smatvec(m->w.w3 + (size_t)l * H * D, m->xb, m->hb2, H, D);
        po_silu(m->hb, H);
        po_vec_mul(m->hb, m->hb, m->hb2, H);
        po_smatvec(m->w.w2 + (size_t)l * D * H, m->hb, m->xb, D, H);
        po_vec_add(m->x, m->x, m->xb, D);
    }
}

/* llama2.c:201-206 = embed (:123-125) + layers + head (:194-198). */
void po_forward(po_model_t *m, int token, int pos) {
    po_embedding_lookup(m->x, m->w.emb, m->c.dim, token);
    forward_layers(m, pos);
    po_rmsnorm(m->x, m->x, m->w.rms_final, m->c.dim);
    po_smatvec(m->w.wcls, m->x, m->logits, m->c.vocab_size, m->c.dim);
}

/* pt.c:267-271 */
int po_forward_step(po_model_t *m, int token) {
    po_forward(m, token, m->pos);
    m->pos++;
    return po_argmax(m->logits, m->c.vocab_size);
}

const float *po_logits(const po_model_t *m) { return m->logits; }
const float *po_residual(const po_model_t *m) { return m->x; }
int po_pos(const po_model_t *m) { return m->pos; }

/* pt_text.c:314-361 with temperature 0 (pt_sample -> argmax, :256-257). */
int po_generate_greedy(po_model_t *m, const int *prompt, int n_prompt,
                       int max_tokens, int *out) {
    if (max_tokens > m->c.seq_len) max_tokens = m->c.seq_len;
    po_reset_kv(m);
    int token = prompt[0], n = 0;
    for (int pos = 0; pos < max_tokens; pos++) {
        po_forward(m, token, pos);
        int sampled = pos >= n_prompt - 1;
        int next = sampled ? po_argmax(m->logits, m->c.vocab_size) : prompt[pos + 1];
        out[n++] = next;
        if (sampled && (next == 1 || next == 2)) break;   /* BOS / EOS stop */
        token = next;
    }
    return n;
}

/* ═══ training — pitorch/train/pt_train.c ════════════════════════════ */

/* pt_train.c:171-329 */
float po_forward_train(po_model_t *m, const int *tokens, int T) {
    const po_config_t *c = &m->c;
    size_t D = c->dim, H = c->hidden_dim, KV = m->kv_dim, V = c->vocab_size;
    int hd = m->head_dim, nh = c->n_heads, kv_mul = nh / c->n_kv_heads;
    int L = c->n_layers;
    float scale = 1.0f / po_sqrtf((float)hd);

    for (int t = 0; t < T; t++)
        po_embedding_lookup(m->res + t * D, m->w.emb, (int)D, tokens[t]);

    for (int l = 0; l < L; l++) {
        float *rin = m->res + (size_t)l * T * D;
        float *rmid = m->res_att + (size_t)l * T * D;
        float *rout = m->res + (size_t)(l + 1) * T * D;
        for (int t = 0; t < T; t++) {
            size_t r = (size_t)l * T + t;
            float *xb = m->xb_att + r * D;
            po_rmsnorm(xb, rin + t * D, m->w.rms_att + l * D, (int)D);
            po_smatvec(m->w.wq + l * D * D, xb, m->aq + r * D, (int)D, (int)D);
            po_smatvec(m->w.wk + l * KV * D, xb, m->ak + r * KV, (int)KV, (int)D);
            po_smatvec(m->w.wv + l * KV * D, xb, m->av + r * KV, (int)KV, (int)D);
            po_rope(m->aq + r * D, m->ak + r * KV, (int)D, hd, t);
        }
        for (int t = 0; t < T; t++) {
            size_t r = (size_t)l * T + t;
            float *ao = m->att_out + r * D;
            for (int h = 0; h < nh; h++) {
                const float *qh = m->aq + r * D + h * hd;
                float *ah = m->aatt + (((size_t)l * nh + h) * T + t) * T;
                size_t ko = (size_t)(h / kv_mul) * hd;
                for (int t2 = 0; t2 <= t; t2++) {
                    const float *kt = m->ak + ((size_t)l * T + t2) * KV + ko;
                    float s = 0.0f;
                    for (int i = 0; i < hd; i++) s += qh[i] * kt[i];
                    ah[t2] = s * scale;
                }
                for (int t2 = t + 1; t2 < T; t2++) ah[t2] = 0.0f;
                po_softmax(ah, t + 1);
                float *oh = ao + h * hd;
                memset(oh, 0, hd * sizeof(float));
                for (int t2 = 0; t2 <= t; t2++) {
                    const float *vt = m->av + ((size_t)l * T + t2) * KV + ko;
                    float a = ah[t2];
                    for (int i = 0; i < hd; i++) oh[i] += a * vt[i];
                }
            }
            po_smatvec(m->w.wo + l * D * D, ao, m->scratch, (int)D, (int)D);
            po_vec_add(rmid + t * D, rin + t * D, m->scratch, (int)D);
        }
        for (int t = 0; t < T; t++) {
            size_t r = (size_t)l * T + t;
            float *xb = m->xb_ffn + r * D;
            po_rmsnorm(xb, rmid + t * D, m->w.rms_ffn + l * D, (int)D);
            float *h1 = m->ahb + r * H, *h3 = m->ahb2 + r * H;
            po_smatvec(m->w.w1 + l * H * D, xb, h1, (int)H, (int)D);
            po_smatvec(m->w.w3 + l * H * D, xb, h3, (int)H, (int)D);
            /* :280-284 — silu as x*sigmoid(x), not x/(1+e^-x) */
            for (size_t i = 0; i < H; i++) {
                float sig = 1.0f / (1.0f + po_expf(-h1[i]));
                m->scratch[i] = (h1[i] * sig) * h3[i];
            }
            po_smatvec(m->w.w2 + l * D * H, m->scratch, rout + t * D, (int)D, (int)H);
            po_vec_add(rout + t * D, rout + t * D, rmid + t * D, (int)D);
        }
    }

    const float *rfin = m->res + (size_t)L * T * D;
    for (int t = 0; t < T; t++) {
        po_rmsnorm(m->x_final + t * D, rfin + t * D, m->w.rms_final, (int)D);
        po_smatvec(m->w.wcls, m->x_final + t * D, m->tlogits + t * V, (int)V, (int)D);
    }
    /* :310-325 */
    float loss = 0.0f;
    for (int t = 0; t < T - 1; t++) {
        const float *lg = m->tlogits + t * V;
        int tgt = tokens[t + 1];
        float mx = lg[0];
        for (size_t v = 1; v < V; v++) if (lg[v] > mx) mx = lg[v];
        float sum = 0.0f;
        for (size_t v = 0; v < V; v++) sum += po_expf(lg[v] - mx);
        loss += -(lg[tgt] - mx - po_logf(sum));
    }
    loss /= (float)(T - 1);
    return loss;
}

void po_zero_grads(po_model_t *m) {
    memset(m->gmem, 0, (size_t)m->n_params * sizeof(float));
}

/* d_x = W^T d_y with a fresh sum (pt_train.c:442-453, accumulate = 0). */
static void bwd_input_fresh(float *d_x, const float *W, const float *d_y,
                            int out_dim, int in_dim) {
    memset(d_x, 0, (size_t)in_dim * sizeof(float));
    po_matmul_backward_input(d_x, W, d_y, out_dim, in_dim);
}

/* pt_train.c:549-866; R = T-1 positions carry a loss signal (:596-605). */
void po_backward(po_model_t *m, const int *tokens, int T) {
    const po_config_t *c = &m->c;
    size_t D = c->dim, H = c->hidden_dim, KV = m->kv_dim, V = c->vocab_size;
    int hd = m->head_dim, nh = c->n_heads, kv_mul = nh / c->n_kv_heads;
    int L = c->n_layers, R = T - 1;
    float scale = 1.0f / po_sqrtf((float)hd);

    memset(m->d_res, 0, (size_t)T * D * sizeof(float));
    float inv_T1 = 1.0f / (float)(T - 1);

    /* :609-621 loss gradient */
    for (int t = 0; t < R; t++) {
        float *dl = m->d_logit_all + t * V;
        const float *lg = m->tlogits + t * V;
        int tgt = tokens[t + 1];
        float mx = lg[0];
        for (size_t v = 1; v < V; v++) if (lg[v] > mx) mx = lg[v];
        float sm = 0.0f;
        for (size_t v = 0; v < V; v++) { dl[v] = po_expf(lg[v] - mx); sm += dl[v]; }
        float inv = 1.0f / sm;
        for (size_t v = 0; v < V; v++) dl[v] *= inv * inv_T1;
        dl[tgt] -= inv_T1;
    }
    /* :625-638 classifier dX + final rmsnorm backward */
    for (int t = 0; t < R; t++) {
        bwd_input_fresh(m->d_xb, m->w.wcls, m->d_logit_all + t * V, (int)V, (int)D);
        po_rmsnorm_backward(m->d_res + t * D, m->g.rms_final, m->d_xb,
                            m->res + (size_t)L * T * D + t * D, m->w.rms_final, (int)D);
    }
    /* :651 classifier dW */
    po_matmul_backward_weight_batched(m->g.wcls, m->d_logit_all, m->x_final, (int)V, (int)D, R);

    for (int l = L - 1; l >= 0; l--) {
        /* FFN, :691-750 */
        for (int t = 0; t < R; t++) {
            size_t r = (size_t)l * T + t;
            float *drt = m->d_res + t * D;
            const float *h1 = m->ahb + r * H, *h3 = m->ahb2 + r * H;
            float *sh = m->sh_all + t * H;
            for (size_t i = 0; i < H; i++) {
                float sig = 1.0f / (1.0f + po_expf(-h1[i]));
                sh[i] = (h1[i] * sig) * h3[i];
            }
            memcpy(m->drt_ffn_all + t * D, drt, D * sizeof(float));
            bwd_input_fresh(m->d_hid, m->w.w2 + l * D * H, drt, (int)D, (int)H);
            for (size_t i = 0; i < H; i++) {
                float sig = 1.0f / (1.0f + po_expf(-h1[i]));
                float sv = h1[i] * sig;
                float ds = m->d_hid[i] * h3[i];
                m->d_hid2[i] = m->d_hid[i] * sv;
                m->d_hid[i] = ds * sig * (1.0f + h1[i] * (1.0f - sig));
            }
            memcpy(m->d_hid_all + t * H, m->d_hid, H * sizeof(float));
            memcpy(m->d_hid2_all + t * H, m->d_hid2, H * sizeof(float));
            bwd_input_fresh(m->d_xb, m->w.w1 + l * H * D, m->d_hid, (int)H, (int)D);
            po_matmul_backward_input(m->d_xb, m->w.w3 + l * H * D, m->d_hid2, (int)H, (int)D);
            po_rmsnorm_backward(drt, m->g.rms_ffn + l * D, m->d_xb, m->res_att + r * D,
                                m->w.rms_ffn + l * D, (int)D);
        }
        po_matmul_backward_weight_batched(m->g.w2 + l * D * H, m->drt_ffn_all, m->sh_all,
                                          (int)D, (int)H, R);
        po_matmul_backward_weight_batched(m->g.w1 + l * H * D, m->d_hid_all,
                                          m->xb_ffn + (size_t)l * T * D, (int)H, (int)D, R);
        po_matmul_backward_weight_batched(m->g.w3 + l * H * D, m->d_hid2_all,
                                          m->xb_ffn + (size_t)l * T * D, (int)H, (int)D, R);

        /* Wo, :757-771 */
        memset(m->d_aout, 0, (size_t)T * D * sizeof(float));
        for (int t = 0; t < R; t++) {
            float *drt = m->d_res + t * D;
            po_matmul_backward_input(m->d_aout + t * D, m->w.wo + l * D * D, drt, (int)D, (int)D);
            memcpy(m->drt_wo_all + t * D, drt, D * sizeof(float));
        }
        po_matmul_backward_weight_batched(m->g.wo + l * D * D, m->drt_wo_all,
                                          m->att_out + (size_t)l * T * D, (int)D, (int)D, R);

        /* attention, :776-812 */
        memset(m->d_q, 0, (size_t)T * D * sizeof(float));
        memset(m->d_k, 0, (size_t)T * KV * sizeof(float));
        memset(m->d_v, 0, (size_t)T * KV * sizeof(float));
        for (int t = 0; t < R; t++) {
            for (int h = 0; h < nh; h++) {
                const float *dao = m->d_aout + t * D + h * hd;
                const float *ah = m->aatt + (((size_t)l * nh + h) * T + t) * T;
                size_t ko = (size_t)(h / kv_mul) * hd;
                memset(m->d_att_s, 0, (size_t)T * sizeof(float));
                for (int t2 = 0; t2 <= t; t2++) {
                    const float *vh = m->av + ((size_t)l * T + t2) * KV + ko;
                    float aw = ah[t2];
                    for (int i = 0; i < hd; i++) {
                        m->d_att_s[t2] += dao[i] * vh[i];
                        m->d_v[t2 * KV + ko + i] += aw * dao[i];
                    }
                }
                memset(m->d_pre_sm, 0, (size_t)T * sizeof(float));
                po_softmax_backward(m->d_pre_sm, m->d_att_s, ah, t + 1);
                const float *qh = m->aq + ((size_t)l * T + t) * D + h * hd;
                for (int t2 = 0; t2 <= t; t2++) {
                    const float *kh = m->ak + ((size_t)l * T + t2) * KV + ko;
                    float ds = m->d_pre_sm[t2] * scale;
                    for (int i = 0; i < hd; i++) {
                        m->d_q[t * D + h * hd + i] += ds * kh[i];
                        m->d_k[t2 * KV + ko + i] += ds * qh[i];
                    }
                }
            }
        }

        /* RoPE + QKV + attention rmsnorm, :818-852 */
        for (int t = 0; t < R; t++) {
            memset(m->d_qpre, 0, D * sizeof(float));
            memset(m->d_kpre, 0, KV * sizeof(float));
            po_rope_backward(m->d_qpre, m->d_kpre, m->d_q + t * D, m->d_k + t * KV,
                             (int)D, hd, t);
            bwd_input_fresh(m->d_xb, m->w.wq + l * D * D, m->d_qpre, (int)D, (int)D);
            po_matmul_backward_input(m->d_xb, m->w.wk + l * KV * D, m->d_kpre, (int)KV, (int)D);
            po_matmul_backward_input(m->d_xb, m->w.wv + l * KV * D, m->d_v + t * KV, (int)KV, (int)D);
            memcpy(m->d_qpre_all + t * D, m->d_qpre, D * sizeof(float));
            memcpy(m->d_kpre_all + t * KV, m->d_kpre, KV * sizeof(float));
            po_rmsnorm_backward(m->d_res + t * D, m->g.rms_att + l * D, m->d_xb,
                                m->res + ((size_t)l * T + t) * D, m->w.rms_att + l * D, (int)D);
        }
        const float *xa = m->xb_att + (size_t)l * T * D;
        po_matmul_backward_weight_batched(m->g.wq + l * D * D, m->d_qpre_all, xa, (int)D, (int)D, R);
        po_matmul_backward_weight_batched(m->g.wk + l * KV * D, m->d_kpre_all, xa, (int)KV, (int)D, R);
        po_matmul_backward_weight_batched(m->g.wv + l * KV * D, m->d_v, xa, (int)KV, (int)D, R);
    }

    /* :862-863 */
    for (int t = 0; t < R; t++)
        po_embedding_backward(m->g.emb, m->d_res + t * D, (int)D, tokens[t]);
}

/* pt_train.c:870-896: w -= lr*g per tensor; a tied wcls is updated once. */
static void sgd(float *w, const float *g, size_t n, float lr) {
    for (size_t i = 0; i < n; i++) w[i] -= lr * g[i];
}

void po_sgd_update(po_model_t *m, float lr) {
    const po_config_t *c = &m->c;
    size_t D = c->dim, H = c->hidden_dim, L = c->n_layers, KV = m->kv_dim, V = c->vocab_size;
    sgd(m->w.emb, m->g.emb, V * D, lr);
    sgd(m->w.rms_att, m->g.rms_att, L * D, lr);
    sgd(m->w.wq, m->g.wq, L * D * D, lr);
    sgd(m->w.wk, m->g.wk, L * KV * D, lr);
    sgd(m->w.wv, m->g.wv, L * KV * D, lr);
    sgd(m->w.wo, m->g.wo, L * D * D, lr);
    sgd(m->w.rms_ffn, m->g.rms_ffn, L * D, lr);
    sgd(m->w.w1, m->g.w1, L * H * D, lr);
    sgd(m->w.w2, m->g.w2, L * D * H, lr);
    sgd(m->w.w3, m->g.w3, L * H * D, lr);
    sgd(m->w.rms_final, m->g.rms_final, D, lr);
    if (m->w.wcls != m->w.emb) sgd(m->w.wcls, m->g.wcls, V * D, lr);
}

/* pt.c:339-364 */
float po_train_step(po_model_t *m, const int *tokens, int T, float lr) {
    po_zero_grads(m);
    float loss = po_forward_train(m, tokens, T);
    po_backward(m, tokens, T);
    po_sgd_update(m, lr);
    return loss;
}

const float *po_grads(const po_model_t *m, int *n) { if (n) *n = m->n_params; return m->gmem; }
const float *po_train_logits(const po_model_t *m) { return m->tlogits; }
const float *po_train_x_final(const po_model_t *m) { return m->x_final; }
