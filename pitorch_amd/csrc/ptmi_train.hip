// Device-resident training step: pt_train_step (pitorch/pt.c:339-364) =
// zero grads, pt_forward_train (pitorch/train/pt_train.c:171-329),
// pt_backward (:549-866), pt_sgd_update (:870-896), with every projection
// as an fp32 MFMA GEMM over all T positions:
//   forward    Y[T,out]  = X[T,in] . W^T            (NT)
//   backward   dX[R,in]  = dY[R,out] . W            (NN)
//              dW[out,in] += dY[R,out]^T . X[R,in]  (TN)
// with R = T-1 rows (the last position carries no loss, pt_train.c:596-605).
// The device weight layout fuses [wq;wk;wv] and row-interleaves [w1|w3],
// so QKV and w1|w3 are one GEMM each in both directions.
//
// Non-GEMM ops follow the reference's arithmetic order: reductions that are
// short (RMSNorm sums over dim, attention softmax sums over positions,
// attention backward dot products) run sequentially in one lane, exactly as
// the reference loops do; per-column gradient accumulations over positions
// run in ascending t like the reference.  Only the GEMMs (and the 32000-wide
// loss softmax sums) reorder additions.
#include "ptmi_model.h"

#include <cmath>
#include <cstring>
#include <new>

namespace ptmi {

struct TrainState {
    int T_max = 0;
    float *mem = nullptr;
    int *tok = nullptr;
    float *res, *res_att, *xb_att, *qkv, *att, *att_out, *xb_ffn, *h13, *sh, *x_final, *logits;
    float *gmem;
    float *d_res, *d_xb, *d_sh, *d_h13, *d_aout, *d_q, *d_k, *d_v, *d_qkv, *ds, *row_inv, *row_loss, *loss;
    float *ws;
    size_t ws_floats = 0;
};

namespace {

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ── forward kernels ──────────────────────────────────────────────────────

__global__ void k_embed_rows(const int *tok, const float *emb, float *out, int D) {   // pt_train.c:189-191
    const int t = blockIdx.x;
    const float *src = emb + (long)tok[t] * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) out[(long)t * D + i] = src[i];
}

// rmsnorm (pt_ops.c:5-12) per row; the sum of squares is one sequential
// chain as in the reference.
__global__ void k_rmsnorm_rows(const float *in, const float *w, float *out, int D) {
    __shared__ float inv_s;
    const float *x = in + (long)blockIdx.x * D;
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (int i = 0; i < D; i++) ss += x[i] * x[i];
        inv_s = 1.0f / d_sqrtf(ss / D + 1e-5f);
    }
    __syncthreads();
    const float inv = inv_s;
    for (int i = threadIdx.x; i < D; i += blockDim.x) out[(long)blockIdx.x * D + i] = x[i] * inv * w[i];
}

// rope (pt_ops.c:33-49) on the q and k columns of each position's qkv row.
__global__ void k_rope_rows(float *qkv, int T, int D, int QS, int hd) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int pairs = D / 2;
    if (idx >= (long)T * pairs) return;
    const int t = (int)(idx / pairs), i = 2 * (int)(idx % pairs);
    float c, s;
    d_rope_cs(i, hd, t, &c, &s);
    float *q = qkv + (long)t * QS + i, *k = q + D;
    const float q0 = q[0], q1 = q[1], k0 = k[0], k1 = k[1];
    q[0] = q0 * c - q1 * s;
    q[1] = q0 * s + q1 * c;
    k[0] = k0 * c - k1 * s;
    k[1] = k0 * s + k1 * c;
}

// Causal attention for one (position t, head h): pt_train.c:224-255.
__global__ void k_attn_fwd(const float *qkv, float *att, float *att_out, int T, int D, int QS, int KV, int hd,
                           int kv_mul, float scale) {
    extern __shared__ float sc[];
    __shared__ float inv_s;
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const float *q = qkv + (long)t * QS + h * hd;
    const int ko = D + (h / kv_mul) * hd, vo = D + KV + (h / kv_mul) * hd;
    for (int t2 = tid; t2 <= t; t2 += blockDim.x) {
        const float *k = qkv + (long)t2 * QS + ko;
        float s = 0.0f;
        for (int i = 0; i < hd; i++) s += q[i] * k[i];
        sc[t2] = s * scale;
    }
    __syncthreads();
    if (tid == 0) {
        float mx = sc[0];
        for (int t2 = 1; t2 <= t; t2++) if (sc[t2] > mx) mx = sc[t2];
        inv_s = mx;
    }
    __syncthreads();
    const float mx = inv_s;
    for (int t2 = tid; t2 <= t; t2 += blockDim.x) sc[t2] = d_expf(sc[t2] - mx);
    __syncthreads();
    if (tid == 0) {
        float sum = 0.0f;
        for (int t2 = 0; t2 <= t; t2++) sum += sc[t2];
        inv_s = 1.0f / sum;
    }
    __syncthreads();
    const float inv = inv_s;
    float *arow = att + ((long)h * T + t) * T;
    for (int t2 = tid; t2 < T; t2 += blockDim.x) {
        const float a = t2 <= t ? sc[t2] * inv : 0.0f;
        arow[t2] = a;
        if (t2 <= t) sc[t2] = a;
    }
    __syncthreads();
    for (int i = tid; i < hd; i += blockDim.x) {
        float o = 0.0f;
        for (int t2 = 0; t2 <= t; t2++) o += sc[t2] * qkv[(long)t2 * QS + vo + i];
        att_out[(long)t * D + h * hd + i] = o;
    }
}

// silu(h1)*h3 in the training form (h1*sigmoid(h1))*h3, pt_train.c:280-284.
__global__ void k_swiglu_fwd(const float *h13, float *sh, long n, int H) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const long t = idx / H, i = idx % H;
    const float h1 = h13[t * 2 * H + 2 * i], h3 = h13[t * 2 * H + 2 * i + 1];
    const float sig = 1.0f / (1.0f + d_expf(-h1));
    sh[idx] = (h1 * sig) * h3;
}

// Cross-entropy row t < T-1 (pt_train.c:310-325) and, in place, its loss
// gradient (pt_train.c:609-621); the last row's gradient is zero.
__global__ __launch_bounds__(256) void k_loss_rows(float *lg_dl, const int *tok, int T, int V, float inv_T1,
                                                   float *row_loss) {
    __shared__ float red[256];
    __shared__ float bcast[2];
    const int t = blockIdx.x, tid = threadIdx.x;
    float *row = lg_dl + (long)t * V;
    if (t == T - 1) {
        for (int v = tid; v < V; v += 256) row[v] = 0.0f;
        return;
    }
    const int target = tok[t + 1];
    float mx = -INFINITY;
    for (int v = tid; v < V; v += 256) mx = fmaxf(mx, row[v]);
    red[tid] = mx;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) red[tid] = fmaxf(red[tid], red[tid + s]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float sum = 0.0f;
    for (int v = tid; v < V; v += 256) sum += d_expf(row[v] - mx);
    red[tid] = sum;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (tid < s) red[tid] += red[tid + s];
        __syncthreads();
    }
    if (tid == 0) {
        sum = red[0];
        row_loss[t] = -(row[target] - mx - d_logf(sum));
        bcast[0] = 1.0f / sum;
    }
    __syncthreads();
    const float scale = bcast[0] * inv_T1;
    for (int v = tid; v < V; v += 256) {
        float d = d_expf(row[v] - mx) * scale;
        if (v == target) d -= inv_T1;
        row[v] = d;
    }
}

__global__ void k_loss_reduce(const float *row_loss, int T, float *loss) {
    float l = 0.0f;
    for (int t = 0; t < T - 1; t++) l += row_loss[t];
    *loss = l / (float)(T - 1);
}

// ── backward kernels ─────────────────────────────────────────────────────

// rmsnorm_backward (pt_backward_ops.c:4-30), the d_x half, per row.
__global__ void k_rmsnorm_bwd_rows(float *d_x, const float *d_o, const float *x, const float *w, float *inv_out,
                                   int D) {
    __shared__ float sh_inv, sh_c;
    const long r = (long)blockIdx.x * D;
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (int i = 0; i < D; i++) ss += x[r + i] * x[r + i];
        ss = ss / D + 1e-5f;
        const float inv = 1.0f / d_sqrtf(ss);
        float dot = 0.0f;
        for (int i = 0; i < D; i++) dot += d_o[r + i] * w[i] * x[r + i];
        const float coeff = inv * inv * inv / (float)D;
        sh_inv = inv;
        sh_c = coeff * dot;
        inv_out[blockIdx.x] = inv;
    }
    __syncthreads();
    const float inv = sh_inv, cd = sh_c;
    for (int i = threadIdx.x; i < D; i += blockDim.x) d_x[r + i] += inv * d_o[r + i] * w[i] - cd * x[r + i];
}

// The d_w half: d_w[i] += d_o[t][i]*x[t][i]*inv[t], t ascending.
__global__ void k_rmsnorm_bwd_dw(float *d_w, const float *d_o, const float *x, const float *inv, int R, int D) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= D) return;
    float acc = d_w[i];
    for (int t = 0; t < R; t++) acc += d_o[(long)t * D + i] * x[(long)t * D + i] * inv[t];
    d_w[i] = acc;
}

// silu*gate backward (pt_train.c:696-721) into interleaved [d_hid | d_hid2]
// columns matching the w1|w3 row interleave, plus sh for dW2.
__global__ void k_swiglu_bwd(const float *h13, const float *d_sh, float *d_h13, float *sh, long n, int H) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const long t = idx / H, i = idx % H;
    const float h1 = h13[t * 2 * H + 2 * i], h3 = h13[t * 2 * H + 2 * i + 1];
    const float sig = 1.0f / (1.0f + d_expf(-h1));
    const float silu_val = h1 * sig;
    sh[idx] = silu_val * h3;
    const float dh = d_sh[idx];
    const float d_silu = dh * h3;
    d_h13[t * 2 * H + 2 * i + 1] = dh * silu_val;
    d_h13[t * 2 * H + 2 * i] = d_silu * sig * (1.0f + h1 * (1.0f - sig));
}

// Attention backward, row half (pt_train.c:780-811): for (t < R, head h):
// d_att_s, the softmax backward dot, ds = d_pre*scale (kept for the column
// half) and d_q[t] = sum_t2 ds[t2] k[t2].
__global__ void k_attn_bwd_rows(const float *qkv, const float *att, const float *d_aout, float *ds, float *d_q,
                                int T, int D, int QS, int KV, int hd, int kv_mul, float scale) {
    extern __shared__ float sm[];
    float *das = sm, *dpre = sm + T;
    __shared__ float dot_s;
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const float *dao = d_aout + (long)t * D + h * hd;
    const float *arow = att + ((long)h * T + t) * T;
    const int ko = D + (h / kv_mul) * hd, vo = D + KV + (h / kv_mul) * hd;
    for (int t2 = tid; t2 <= t; t2 += blockDim.x) {
        const float *v = qkv + (long)t2 * QS + vo;
        float s = 0.0f;
        for (int i = 0; i < hd; i++) s += dao[i] * v[i];
        das[t2] = s;
    }
    __syncthreads();
    if (tid == 0) {
        float dot = 0.0f;
        for (int t2 = 0; t2 <= t; t2++) dot += das[t2] * arow[t2];
        dot_s = dot;
    }
    __syncthreads();
    const float dot = dot_s;
    float *dsrow = ds + ((long)h * T + t) * T;
    for (int t2 = tid; t2 <= t; t2 += blockDim.x) {
        const float d = arow[t2] * (das[t2] - dot) * scale;
        dpre[t2] = d;
        dsrow[t2] = d;
    }
    __syncthreads();
    for (int i = tid; i < hd; i += blockDim.x) {
        float acc = 0.0f;
        for (int t2 = 0; t2 <= t; t2++) acc += dpre[t2] * qkv[(long)t2 * QS + ko + i];
        d_q[(long)t * D + h * hd + i] = acc;
    }
}

// Attention backward, column half: for (t2 < R, head h), t ascending:
// d_v[t2] = sum_t att[t][t2] d_aout[t],  d_k[t2] = sum_t ds[t][t2] q[t].
__global__ void k_attn_bwd_cols(const float *qkv, const float *att, const float *ds, const float *d_aout, float *d_k,
                                float *d_v, int T, int R, int D, int QS, int KV, int hd, int kv_mul) {
    const int t2 = blockIdx.x, h = blockIdx.y;
    const int kvo = (h / kv_mul) * hd;
    for (int i = threadIdx.x; i < hd; i += blockDim.x) {
        float dv = 0.0f, dk = 0.0f;
        for (int t = t2; t < R; t++) {
            dv += att[((long)h * T + t) * T + t2] * d_aout[(long)t * D + h * hd + i];
            dk += ds[((long)h * T + t) * T + t2] * qkv[(long)t * QS + h * hd + i];
        }
        d_v[(long)t2 * KV + kvo + i] = dv;
        d_k[(long)t2 * KV + kvo + i] = dk;
    }
}

// rope_backward (pt_backward_ops.c:52-69) of d_q, d_k, packed with d_v into
// the fused [dq | dk | dv] row used by the QKV GEMMs.
__global__ void k_rope_bwd_pack(const float *d_q, const float *d_k, const float *d_v, float *d_qkv, int R, int D,
                                int KV, int QS, int hd) {
    const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const int pairs = D / 2;
    if (idx >= (long)R * pairs) return;
    const int t = (int)(idx / pairs), i = 2 * (int)(idx % pairs);
    float c, s;
    d_rope_cs(i, hd, t, &c, &s);
    const float q0 = d_q[(long)t * D + i], q1 = d_q[(long)t * D + i + 1];
    const float k0 = d_k[(long)t * KV + i], k1 = d_k[(long)t * KV + i + 1];
    float *o = d_qkv + (long)t * QS;
    o[i] = q0 * c + q1 * s;
    o[i + 1] = -q0 * s + q1 * c;
    o[D + i] = k0 * c + k1 * s;
    o[D + i + 1] = -k0 * s + k1 * c;
    o[D + KV + i] = d_v[(long)t * KV + i];
    o[D + KV + i + 1] = d_v[(long)t * KV + i + 1];
}

// embedding_backward (pt_backward_ops.c:90-95) for t ascending, per column.
__global__ void k_embed_bwd(const int *tok, const float *d_res, float *g_emb, int R, int D) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= D) return;
    for (int t = 0; t < R; t++) g_emb[(long)tok[t] * D + j] += d_res[(long)t * D + j];
}

// sgd_step (pt_train.c:870-873) over the whole device weight buffer.
__global__ void k_sgd(float *w, const float *g, float lr, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) w[i] -= lr * g[i];
}

inline unsigned blocks_for(long n, int b) { return (unsigned)((n + b - 1) / b); }

float host_scale(int head_dim) {   // 1/pt_sqrtf(hd), pt_train.c:182
    const float x = (float)head_dim;
    uint32_t u;
    memcpy(&u, &x, 4);
    u = 0x1fbd1df5u + (u >> 1);
    float y;
    memcpy(&y, &u, 4);
    for (int i = 0; i < 3; i++) y = 0.5f * (y + x / y);
    return 1.0f / y;
}

}  // namespace

int train_create(ptmi_model *m) {
    const Config &c = m->c;
    if (c.kv_dim != c.dim)
        return set_error(PTMI_ERR_ARG, "training needs n_kv_heads == n_heads (the reference's rope spans dim)");
    TrainState *ts = new TrainState();
    const size_t T = m->max_T, D = c.dim, H = c.hidden, L = c.n_layers, V = c.vocab, KV = c.kv_dim;
    const size_t NH = c.n_heads, QS = D + 2 * KV;
    ts->T_max = (int)T;
    ts->ws_floats = (size_t)8 << 20;
    size_t sizes[] = {
        (L + 1) * T * D, L * T * D, L * T * D, L * T * QS, L * NH * T * T, L * T * D, L * T * D, L * T * 2 * H,
        T * H, T * D, T * V,                                   // forward
        m->res->mem_floats,                                    // grads
        T * D, T * D, T * H, T * 2 * H, T * D, T * D, T * KV, T * KV, T * QS, NH * T * T, T, T, 64,
        ts->ws_floats, T};
    float **dst[] = {&ts->res, &ts->res_att, &ts->xb_att, &ts->qkv, &ts->att, &ts->att_out, &ts->xb_ffn, &ts->h13,
                     &ts->sh, &ts->x_final, &ts->logits, &ts->gmem, &ts->d_res, &ts->d_xb, &ts->d_sh, &ts->d_h13,
                     &ts->d_aout, &ts->d_q, &ts->d_k, &ts->d_v, &ts->d_qkv, &ts->ds, &ts->row_inv, &ts->row_loss,
                     &ts->loss, &ts->ws, (float **)&ts->tok};
    const int nbuf = (int)(sizeof(sizes) / sizeof(sizes[0]));
    size_t total = 0;
    for (int i = 0; i < nbuf; i++) total += align_up(sizes[i], 64);
    hipError_t e = hipMalloc(&ts->mem, total * sizeof(float));
    if (e != hipSuccess) { delete ts; return hip_check(e, "hipMalloc(training state)"); }
    size_t o = 0;
    for (int i = 0; i < nbuf; i++) { *dst[i] = ts->mem + o; o += align_up(sizes[i], 64); }
    e = hipMemsetAsync(ts->mem, 0, total * sizeof(float), lib_stream());
    if (e == hipSuccess) e = hipStreamSynchronize(lib_stream());
    if (e != hipSuccess) { (void)hipFree(ts->mem); delete ts; return hip_check(e, "zero training state"); }
    m->train = ts;
    return PTMI_OK;
}

void train_destroy(ptmi_model *m) {
    if (!m->train) return;
    (void)hipFree(m->train->mem);
    delete m->train;
    m->train = nullptr;
}

namespace {

int gemm(hipStream_t s, TrainState *ts, int op, const float *A, long lda, const float *B, long ldb, float *C, long ldc,
         int M, int N, int K, int acc) {
    return launch_gemm(op, A, lda, B, ldb, C, ldc, M, N, K, acc, ts->ws, ts->ws_floats, s);
}

int rmsnorm_bwd(hipStream_t s, TrainState *ts, float *d_x, const float *d_o, const float *x, const float *w,
                float *d_w, int R, int D) {
    hipLaunchKernelGGL(k_rmsnorm_bwd_rows, dim3(R), dim3(256), 0, s, d_x, d_o, x, w, ts->row_inv, D);
    hipLaunchKernelGGL(k_rmsnorm_bwd_dw, dim3(blocks_for(D, 256)), dim3(256), 0, s, d_w, d_o, x, ts->row_inv, R, D);
    PTMI_HIP(hipGetLastError());
    return PTMI_OK;
}

int enqueue_train(ptmi_model *m, int T, float lr, hipStream_t s) {
    TrainState *ts = m->train;
    const Resident *r = m->res;
    const Config &c = m->c;
    const int D = c.dim, H = c.hidden, L = c.n_layers, V = c.vocab, KV = c.kv_dim, NH = c.n_heads, hd = c.head_dim;
    const int QS = D + 2 * KV, R = T - 1, kv_mul = c.n_heads / c.n_kv_heads;
    const float scale = host_scale(hd);
    const long TD = (long)T * D;
    auto G = [&](const float *p) { return ts->gmem + (p - r->mem); };   // grad of a weight tensor
    int st;
    const size_t att_lds = (size_t)T * sizeof(float);

    PTMI_HIP(hipMemsetAsync(ts->gmem, 0, r->mem_floats * sizeof(float), s));        // pt_zero_grads
    // ── forward ──
    hipLaunchKernelGGL(k_embed_rows, dim3(T), dim3(256), 0, s, ts->tok, r->emb, ts->res, D);
    for (int l = 0; l < L; l++) {
        float *rin = ts->res + l * TD, *rmid = ts->res_att + l * TD, *rout = ts->res + (l + 1) * TD;
        float *xa = ts->xb_att + l * TD, *qkv = ts->qkv + (long)l * T * QS, *att = ts->att + (long)l * NH * T * T;
        float *ao = ts->att_out + l * TD, *xf = ts->xb_ffn + l * TD, *h13 = ts->h13 + (long)l * T * 2 * H;
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(T), dim3(256), 0, s, rin, r->rms_att + (long)l * D, xa, D);
        if ((st = gemm(s, ts, 2, xa, D, r->wqkv + (long)l * QS * D, D, qkv, QS, T, QS, D, 0))) return st;
        hipLaunchKernelGGL(k_rope_rows, dim3(blocks_for((long)T * D / 2, 256)), dim3(256), 0, s, qkv, T, D, QS, hd);
        hipLaunchKernelGGL(k_attn_fwd, dim3(T, NH), dim3(64), att_lds, s, qkv, att, ao, T, D, QS, KV, hd, kv_mul, scale);
        PTMI_HIP(hipMemcpyAsync(rmid, rin, TD * sizeof(float), hipMemcpyDeviceToDevice, s));
        if ((st = gemm(s, ts, 2, ao, D, r->wo + (long)l * D * D, D, rmid, D, T, D, D, 1))) return st;
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(T), dim3(256), 0, s, rmid, r->rms_ffn + (long)l * D, xf, D);
        if ((st = gemm(s, ts, 2, xf, D, r->w13 + (long)l * 2 * H * D, D, h13, 2 * H, T, 2 * H, D, 0))) return st;
        hipLaunchKernelGGL(k_swiglu_fwd, dim3(blocks_for((long)T * H, 256)), dim3(256), 0, s, h13, ts->sh, (long)T * H, H);
        PTMI_HIP(hipMemcpyAsync(rout, rmid, TD * sizeof(float), hipMemcpyDeviceToDevice, s));
        if ((st = gemm(s, ts, 2, ts->sh, H, r->w2 + (long)l * D * H, H, rout, D, T, D, H, 1))) return st;
    }
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3(T), dim3(256), 0, s, ts->res + L * TD, r->rms_final, ts->x_final, D);
    if ((st = gemm(s, ts, 2, ts->x_final, D, r->wcls, D, ts->logits, V, T, V, D, 0))) return st;
    hipLaunchKernelGGL(k_loss_rows, dim3(T), dim3(256), 0, s, ts->logits, ts->tok, T, V, 1.0f / (float)(T - 1),
                       ts->row_loss);
    hipLaunchKernelGGL(k_loss_reduce, dim3(1), dim3(1), 0, s, ts->row_loss, T, ts->loss);
    PTMI_HIP(hipGetLastError());

    // ── backward ── (ts->logits now holds d_logits)
    PTMI_HIP(hipMemsetAsync(ts->d_res, 0, TD * sizeof(float), s));
    if ((st = gemm(s, ts, 0, ts->logits, V, r->wcls, D, ts->d_xb, D, R, D, V, 0))) return st;
    if ((st = rmsnorm_bwd(s, ts, ts->d_res, ts->d_xb, ts->res + L * TD, r->rms_final, G(r->rms_final), R, D))) return st;
    if ((st = gemm(s, ts, 1, ts->logits, V, ts->x_final, D, G(r->wcls), D, V, D, R, 1))) return st;
    for (int l = L - 1; l >= 0; l--) {
        const float *rin = ts->res + l * TD, *rmid = ts->res_att + l * TD;
        const float *xa = ts->xb_att + l * TD, *qkv = ts->qkv + (long)l * T * QS, *att = ts->att + (long)l * NH * T * T;
        const float *ao = ts->att_out + l * TD, *xf = ts->xb_ffn + l * TD, *h13 = ts->h13 + (long)l * T * 2 * H;
        const float *w2 = r->w2 + (long)l * D * H, *w13 = r->w13 + (long)l * 2 * H * D;
        const float *wo = r->wo + (long)l * D * D, *wqkv = r->wqkv + (long)l * QS * D;
        // FFN
        if ((st = gemm(s, ts, 0, ts->d_res, D, w2, H, ts->d_sh, H, R, H, D, 0))) return st;
        hipLaunchKernelGGL(k_swiglu_bwd, dim3(blocks_for((long)R * H, 256)), dim3(256), 0, s, h13, ts->d_sh, ts->d_h13,
                           ts->sh, (long)R * H, H);
        if ((st = gemm(s, ts, 1, ts->d_res, D, ts->sh, H, G(w2), H, D, H, R, 1))) return st;
        if ((st = gemm(s, ts, 0, ts->d_h13, 2 * H, w13, D, ts->d_xb, D, R, D, 2 * H, 0))) return st;
        if ((st = gemm(s, ts, 1, ts->d_h13, 2 * H, xf, D, G(w13), D, 2 * H, D, R, 1))) return st;
        if ((st = rmsnorm_bwd(s, ts, ts->d_res, ts->d_xb, rmid, r->rms_ffn + (long)l * D,
                              G(r->rms_ffn + (long)l * D), R, D))) return st;
        // Wo
        if ((st = gemm(s, ts, 0, ts->d_res, D, wo, D, ts->d_aout, D, R, D, D, 0))) return st;
        if ((st = gemm(s, ts, 1, ts->d_res, D, ao, D, G(wo), D, D, D, R, 1))) return st;
        // attention
        hipLaunchKernelGGL(k_attn_bwd_rows, dim3(R, NH), dim3(64), 2 * att_lds, s, qkv, att, ts->d_aout, ts->ds, ts->d_q,
                           T, D, QS, KV, hd, kv_mul, scale);
        hipLaunchKernelGGL(k_attn_bwd_cols, dim3(R, NH), dim3(64), 0, s, qkv, att, ts->ds, ts->d_aout, ts->d_k, ts->d_v,
                           T, R, D, QS, KV, hd, kv_mul);
        hipLaunchKernelGGL(k_rope_bwd_pack, dim3(blocks_for((long)R * D / 2, 256)), dim3(256), 0, s, ts->d_q, ts->d_k,
                           ts->d_v, ts->d_qkv, R, D, KV, QS, hd);
        PTMI_HIP(hipGetLastError());
        // QKV
        if ((st = gemm(s, ts, 0, ts->d_qkv, QS, wqkv, D, ts->d_xb, D, R, D, QS, 0))) return st;
        if ((st = gemm(s, ts, 1, ts->d_qkv, QS, xa, D, G(wqkv), D, QS, D, R, 1))) return st;
        if ((st = rmsnorm_bwd(s, ts, ts->d_res, ts->d_xb, rin, r->rms_att + (long)l * D,
                              G(r->rms_att + (long)l * D), R, D))) return st;
    }
    hipLaunchKernelGGL(k_embed_bwd, dim3(blocks_for(D, 256)), dim3(256), 0, s, ts->tok, ts->d_res, G(r->emb), R, D);
    // ── SGD ──
    hipLaunchKernelGGL(k_sgd, dim3(blocks_for((long)r->mem_floats, 256)), dim3(256), 0, s, r->mem, ts->gmem, lr,
                       (long)r->mem_floats);
    PTMI_HIP(hipGetLastError());
    return PTMI_OK;
}

}  // namespace

}  // namespace ptmi

using namespace ptmi;

extern "C" {

int ptmi_model_train_step(ptmi_model_t *m, const int *tokens, int T, float lr, float *loss) {
    if (!m || !tokens) return set_error(PTMI_ERR_ARG, "NULL argument");
    if (!m->train) return set_error(PTMI_ERR_STATE, "model created with max_T = 0 (no training buffers)");
    if (T < 2 || T > m->train->T_max) return set_error(PTMI_ERR_ARG, "T=%d outside [2, max_T=%d]", T, m->train->T_max);
    for (int i = 0; i < T; i++)
        if (tokens[i] < 0 || tokens[i] >= m->c.vocab) return set_error(PTMI_ERR_ARG, "tokens[%d]=%d out of range", i, tokens[i]);
    hipStream_t s = lib_stream();
    PTMI_HIP(hipMemcpyAsync(m->train->tok, tokens, (size_t)T * sizeof(int), hipMemcpyHostToDevice, s));
    int st = enqueue_train(m, T, lr, s);
    if (st) return st;
    float l = 0.0f;
    PTMI_HIP(hipMemcpyAsync(&l, m->train->loss, sizeof(float), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    if (loss) *loss = l;
    return PTMI_OK;
}

// Gradient buffer in pt_grads_t order (pt_train.c:342-370): converted from
// the device layout by the same copy plan as the weights.
int ptmi_model_read_grads(ptmi_model_t *m, float *out, size_t n_floats) {
    if (!m || !out) return set_error(PTMI_ERR_ARG, "NULL argument");
    if (!m->train) return set_error(PTMI_ERR_STATE, "no training buffers");
    Resident *r = m->res;
    const Config &c = r->c;
    const size_t D = c.dim, H = c.hidden, L = c.n_layers, KV = c.kv_dim, V = c.vocab;
    const size_t n = V * D + L * D + L * D * D + 2 * L * KV * D + L * D * D + L * D + 3 * L * H * D + D +
                     (c.shared ? 0 : V * D);
    if (n_floats < n) return set_error(PTMI_ERR_ARG, "buffer holds %zu floats, gradients need %zu", n_floats, n);
    // Reuse the weight download plan: view the grad buffer as a fake resident.
    Resident g = *r;
    g.mem = m->train->gmem;
    auto rebase = [&](float *p) { return g.mem + (p - r->mem); };
    g.emb = rebase(r->emb); g.rms_att = rebase(r->rms_att); g.wqkv = rebase(r->wqkv); g.wo = rebase(r->wo);
    g.rms_ffn = rebase(r->rms_ffn); g.w13 = rebase(r->w13); g.w2 = rebase(r->w2); g.rms_final = rebase(r->rms_final);
    g.wcls = rebase(r->wcls);
    // download into a blob-shaped staging buffer (header + tensors + freq_cis)
    const size_t blob_floats = (r->bytes - 28) / sizeof(float);
    float *stage = new (std::nothrow) float[blob_floats + 7];
    if (!stage) return set_error(PTMI_ERR_OOM, "host staging for gradients");
    memcpy(stage, r->blob, 28);
    int st = download_resident(&g, stage, lib_stream());
    if (st) { delete[] stage; return st; }
    // pt_grads_t order = file order without the freq_cis blocks (tied: no wcls)
    const float *src = (const float *)((const char *)stage + 28);
    const size_t before_freq = r->off_rms_final + D;
    memcpy(out, src, before_freq * sizeof(float));
    if (!c.shared) memcpy(out + before_freq, src + r->off_wcls, V * D * sizeof(float));
    delete[] stage;
    return PTMI_OK;
}

}  // extern "C"
