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
// Non-GEMM ops keep the reference's element-wise arithmetic; their sums
// (RMSNorm squares, softmax sums, column gradient accumulations) are wave
// or block reductions and the attention products run on the matrix cores,
// so their addition order differs from the reference's sequential loops, as
// in the GEMMs.  The embedding gradient keeps the reference's order exactly
// (per token and column, positions ascending).
#include "ptmi_model.h"

#include <cmath>
#include <cstring>
#include <new>
#include <vector>

namespace ptmi {

struct TrainState {
    int T_max = 0;
    float *mem = nullptr;
    int *tok = nullptr;
    float *res, *res_att, *xb_att, *qkv, *att, *att_out, *xb_ffn, *h13, *sh, *x_final, *logits;
    float *gmem;
    // Backward buffers.  What the deferred weight-gradient launches read is
    // written once per step: d_res and d_xb by version (one per RMSNorm
    // backward, 2L+1, plus d_res's zero start), d_h13, sh and d_qkv per
    // layer, the RMSNorm inverse norms per norm.
    float *d_res, *d_xb, *d_sh, *d_h13, *shb, *d_aout, *d_q, *d_k, *d_v, *d_qkv, *ds, *row_inv, *row_loss, *loss;
    // Descriptor tables of the two grouped launches (device; built per T).
    void *dw_desc;
    float *nd_desc;
    int desc_T = 0, dw_tiles = 0, n_dw = 0, dw_vec = 0, dw_cls_tiles = 0;   // entry 0: the classifier
    float *ws;
    size_t ws_floats = 0;
    float *lr;                  // device copy of the step's learning rate (lr_off floats past tok)
    // Pinned host staging: the step's tokens and learning rate laid out as
    // tok .. lr are on the device (one copy in), then the loss (one copy out).
    float *pin = nullptr;
    long lr_off = 0;
    bool pin_busy = false;      // a copy from pin may be in flight (cleared by the step's final synchronisation)
    // Bit t of tok_bits: token t is the input at some position < T-1.  Set by
    // the forward's embedding gather, read by the classifier dW GEMM (which
    // leaves those embedding rows' SGD step to the embedding backward), and
    // cleared by the embedding backward, so it is all zero between steps.
    unsigned *tok_bits;
    // The step for one T, captured once (PTMI_TRAIN_EAGER=1: plain launches).
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int graph_T = 0;
    bool eager = false;
    // Which RMSNorm kinds run fused into the next GEMM where launch_gemm can:
    // bit k-1 for GemmNorm kind k (PTMI_TRAIN_FUSE_NORM overrides)
    int fuse_norm = 5;
};

namespace {

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ── block reductions (every thread gets the result) ──────────────────────

template <int NW>
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    __syncthreads();                       // red may still be read by a previous call
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) s += red[w];
    return s;
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float *red) {
    v = group_max<64>(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) m = fmaxf(m, red[w]);
    return m;
}

// Sum / max over the 64 lanes of a wave, returned to every lane: DPP within
// each row of 16 lanes (quad xor 1, quad xor 2, half-row mirror, row
// mirror), then the four row results read as scalars.  No LDS round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

__device__ __forceinline__ float dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }

// ── forward kernels ──────────────────────────────────────────────────────

// (also marks tok[t] in tok_bits for t < R)
__global__ void k_embed_rows(const int *tok, const float *emb, float *out, int D, unsigned *tok_bits, int R) {
    const int t = blockIdx.x;                                    // pt_train.c:189-191
    if (threadIdx.x == 0 && t < R) atomicOr(&tok_bits[tok[t] >> 5], 1u << (tok[t] & 31));
    const float *src = emb + (long)tok[t] * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) out[(long)t * D + i] = src[i];
}

// rmsnorm (pt_ops.c:5-12) per row.
// With pk.splits > 0 the row x is first completed from split-K partial sums
// of the GEMM that produced it, x = (cin +) sum_z pk.parts[z] (the split-K
// reduction, z ascending), and stored; each thread re-reads only the
// elements it stored.
__global__ __launch_bounds__(256) void k_rmsnorm_rows(float *in, const float *w, float *out, int D, SplitK pk,
                                                      const float *cin) {
    __shared__ float red[4];
    const long r = (long)blockIdx.x * D;
    float *x = in + r;
    if (pk.splits > 0) {                                         // uniform
        for (int i = threadIdx.x; i < D; i += 256) {
            const float v = sum_splits(pk.parts, pk.splits, pk.stride, r + i);
            x[i] = cin ? cin[r + i] + v : v;
        }
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < D; i += 256) ss += x[i] * x[i];
    ss = block_sum<4>(ss, red);
    const float inv = 1.0f / d_sqrtf(ss / D + 1e-5f);
    for (int i = threadIdx.x; i < D; i += 256) out[r + i] = x[i] * inv * w[i];
}

// Attention blocks: 256 threads; G lanes (G*4 >= head_dim) hold one
// position's head row as float4, so a wave covers 64/G positions per load
// and the block 256/G.
constexpr int kAttnThreads = 256;

// Per-position dot products s[t2] = a . B[t2] (B rows at b + t2*ld) for t2
// in [0, n), G lanes per row; lane sub's float4 of `a` is a4.
template <int G>
__device__ __forceinline__ void row_dots(const float *b, long ld, float4 a4, int hd4, int n, float *out, float mul) {
    constexpr int S = kAttnThreads / G;
    const int slot = threadIdx.x / G, sub = threadIdx.x % G;
    const bool has = sub < hd4;
    for (int base = 0; base < n; base += 4 * S) {
        float4 r[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t2 = min(base + u * S + slot, n - 1);
            r[u] = has ? reinterpret_cast<const float4 *>(b + (long)t2 * ld)[sub] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            float v = has ? dot4(a4, r[u]) : 0.0f;
            v = group_sum<G>(v);
            const int t2 = base + u * S + slot;
            if (sub == 0 && t2 < n) out[t2] = v * mul;
        }
    }
}

// o[i] = sum_{t2 < n} w[t2] B[t2][i] for i < hd (B rows at b + t2*ld); the
// 256/G slots take interleaved positions and their partial sums meet in
// LDS `part` (at least (256/G)*hd floats).  Thread i < hd returns o[i].
constexpr int kAttnPart = 1024;   // (256/G) * hd <= 1024 for hd <= 4*G
template <int G>
__device__ __forceinline__ float weighted_rows(const float *b, long ld, const float *w, int hd4, int n, float *part) {
    constexpr int S = kAttnThreads / G;
    const int slot = threadIdx.x / G, sub = threadIdx.x % G;
    const bool has = sub < hd4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int base = 0; base < n; base += 4 * S) {
        float4 r[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t2 = min(base + u * S + slot, n - 1);
            r[u] = has ? reinterpret_cast<const float4 *>(b + (long)t2 * ld)[sub] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t2 = base + u * S + slot;
            const float e = t2 < n ? w[t2] : 0.0f;
            acc.x += e * r[u].x;
            acc.y += e * r[u].y;
            acc.z += e * r[u].z;
            acc.w += e * r[u].w;
        }
    }
    const int hd = 4 * hd4;
    __syncthreads();                      // earlier readers of part are done
    if (has) reinterpret_cast<float4 *>(part + slot * hd)[sub] = acc;
    __syncthreads();
    float o = 0.0f;
    if ((int)threadIdx.x < hd) {
        o = part[threadIdx.x];
        for (int k = 1; k < S; k++) o += part[k * hd + threadIdx.x];
    }
    return o;
}

// Causal attention for one (position t, head h): pt_train.c:224-255.
// Dynamic LDS: sc[T].
template <int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn_fwd(const float *qkv, float *att, float *att_out, int T, int D,
                                                           int QS, int KV, int hd, int kv_mul, float scale) {
    extern __shared__ float sc[];
    __shared__ float part[kAttnPart];
    __shared__ float red[4];
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, hd4 = hd >> 2, sub = tid % G;
    const int ko = D + (h / kv_mul) * hd, vo = D + KV + (h / kv_mul) * hd;
    const float4 q4 = sub < hd4 ? reinterpret_cast<const float4 *>(qkv + (long)t * QS + h * hd)[sub]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
    const int n = t + 1;
    row_dots<G>(qkv + ko, QS, q4, hd4, n, sc, scale);
    __syncthreads();
    float mx = -INFINITY;
    for (int t2 = tid; t2 < n; t2 += kAttnThreads) mx = fmaxf(mx, sc[t2]);
    mx = block_max<4>(mx, red);
    float sum = 0.0f;
    for (int t2 = tid; t2 < n; t2 += kAttnThreads) {
        const float e = d_expf(sc[t2] - mx);
        sc[t2] = e;
        sum += e;
    }
    sum = block_sum<4>(sum, red);
    const float inv = 1.0f / sum;
    float *arow = att + ((long)h * T + t) * T;
    for (int t2 = tid; t2 < T; t2 += kAttnThreads) {
        const float a = t2 < n ? sc[t2] * inv : 0.0f;
        arow[t2] = a;
        if (t2 < n) sc[t2] = a;
    }
    __syncthreads();
    const float o = weighted_rows<G>(qkv + vo, QS, sc, hd4, n, part);
    if (tid < hd) att_out[(long)t * D + h * hd + tid] = o;
}

// Cross-entropy row t < T-1 (pt_train.c:310-325) and, in place, its loss
// gradient (pt_train.c:609-621); the last row's gradient is zero.  Pass 1
// keeps a running (max, sum of e^(x-max)) per thread, merged over the block.
constexpr int kLossThreads = 1024;
__global__ __launch_bounds__(kLossThreads) void k_loss_rows(float *lg_dl, const int *tok, int T, int V, float inv_T1,
                                                            float *row_loss) {
    __shared__ float red[kLossThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x;
    float *row = lg_dl + (long)t * V;
    const bool vec = (V % 4) == 0;
    const int n4 = vec ? V / 4 : 0;
    float4 *row4 = reinterpret_cast<float4 *>(row);
    if (t == T - 1) {
        for (int v = tid; v < n4; v += kLossThreads) row4[v] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int v = 4 * n4 + tid; v < V; v += kLossThreads) row[v] = 0.0f;
        return;
    }
    const int target = tok[t + 1];
    float m = -INFINITY, s = 0.0f;
    auto add = [&](float x) {
        if (x > m) {
            s = s * d_expf(m - x) + 1.0f;      // e^(-inf) = 0 on the first element
            m = x;
        } else {
            s += d_expf(x - m);
        }
    };
    for (int v = tid; v < n4; v += kLossThreads) {
        const float4 x = row4[v];
        add(x.x); add(x.y); add(x.z); add(x.w);
    }
    for (int v = 4 * n4 + tid; v < V; v += kLossThreads) add(row[v]);
    const float mx = block_max<kLossThreads / 64>(m, red);
    const float part = m == -INFINITY ? 0.0f : s * d_expf(m - mx);
    const float sum = block_sum<kLossThreads / 64>(part, red);
    if (tid == 0) row_loss[t] = -(row[target] - mx - d_logf(sum));
    __syncthreads();                           // row[target] is read before it is overwritten
    const float scale = (1.0f / sum) * inv_T1;
    for (int v = tid; v < n4; v += kLossThreads) {
        const float4 x = row4[v];
        float4 d;
        d.x = d_expf(x.x - mx) * scale;
        d.y = d_expf(x.y - mx) * scale;
        d.z = d_expf(x.z - mx) * scale;
        d.w = d_expf(x.w - mx) * scale;
        const int b = 4 * v;
        if (target >= b && target < b + 4) (&d.x)[target - b] -= inv_T1;
        row4[v] = d;
    }
    for (int v = 4 * n4 + tid; v < V; v += kLossThreads) {
        float d = d_expf(row[v] - mx) * scale;
        if (v == target) d -= inv_T1;
        row[v] = d;
    }
}

// The same row loss and gradient with the row held in registers, for rows of
// V % 4 == 0 and V <= 4 * NS * kLossThreads: one read and one write of the
// logits and one exp per element.  The maximum comes first, then the sum of
// e^(x - max) (the reference's loss order, pt_train.c:311-323), and the
// gradient is formed from the kept exps.  Loads are unconditional (clamped
// to the row) and out-of-row slots are dropped by selects.  The gradient
// rows are written with nontemporal stores: a 1024-thread block streaming
// its 128 KB row out with ordinary stores measured 2x slower (a row-copy
// probe: 19.8 vs 9.2 us for 32.8 MB).
template <int NS>
__global__ __launch_bounds__(kLossThreads) void k_loss_rows_reg(float *lg_dl, const int *tok, int T, int V,
                                                                float inv_T1, float *row_loss) {
    __shared__ float red[kLossThreads / 64];
    const int t = blockIdx.x, tid = threadIdx.x, n4 = V / 4;
    float4 *row4 = reinterpret_cast<float4 *>(lg_dl + (long)t * V);
    if (t == T - 1) {
        for (int v = tid; v < n4; v += kLossThreads) row4[v] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const int target = tok[t + 1];
    const float xt = lg_dl[(long)t * V + target];
    float4 x[NS];
#pragma unroll
    for (int i = 0; i < NS; i++) x[i] = row4[min(tid + i * kLossThreads, n4 - 1)];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const float mi = fmaxf(fmaxf(x[i].x, x[i].y), fmaxf(x[i].z, x[i].w));
        m = tid + i * kLossThreads < n4 ? fmaxf(m, mi) : m;
    }
    const float mx = block_max<kLossThreads / 64>(m, red);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NS; i++) {
        x[i].x = d_expf(x[i].x - mx);
        x[i].y = d_expf(x[i].y - mx);
        x[i].z = d_expf(x[i].z - mx);
        x[i].w = d_expf(x[i].w - mx);
        const float si = x[i].x + x[i].y + x[i].z + x[i].w;
        s = tid + i * kLossThreads < n4 ? s + si : s;
    }
    const float sum = block_sum<kLossThreads / 64>(s, red);
    if (tid == 0) row_loss[t] = -(xt - mx - d_logf(sum));
    const float scale = (1.0f / sum) * inv_T1;
    typedef float fx4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < NS; i++) {
        const int v = tid + i * kLossThreads;
        if (v < n4) {
            fx4 d = {x[i].x * scale, x[i].y * scale, x[i].z * scale, x[i].w * scale};
            const int b = 4 * v;
            d.x = target == b ? d.x - inv_T1 : d.x;
            d.y = target == b + 1 ? d.y - inv_T1 : d.y;
            d.z = target == b + 2 ? d.z - inv_T1 : d.z;
            d.w = target == b + 3 ? d.w - inv_T1 : d.w;
            __builtin_nontemporal_store(d, reinterpret_cast<fx4 *>(row4) + v);
        }
    }
}

// loss = mean of the R = T-1 row losses (pt_train.c:323-326), one block of
// NW waves.
template <int NW>
__device__ __forceinline__ void loss_mean_block(const float *row_loss, int R, float *loss) {
    __shared__ float red[NW];
    float l = 0.0f;
    for (int t = threadIdx.x; t < R; t += 64 * NW) l += row_loss[t];
    l = block_sum<NW>(l, red);
    if (threadIdx.x == 0) *loss = l / (float)R;
}

// ── backward kernels ─────────────────────────────────────────────────────

// rmsnorm_backward (pt_backward_ops.c:4-30), the d_x half, per row:
// d_out = d_in + (the reference's in-place d_x += term).
// With pk.splits > 0, d_o is first completed from the split-K partial sums
// of the GEMM that produced it (z ascending) and stored.
__global__ __launch_bounds__(256) void k_rmsnorm_bwd_rows(float *d_out, const float *d_in, float *d_o,
                                                          const float *x, const float *w, float *inv_out, int D,
                                                          SplitK pk) {
    __shared__ float red[4];
    const long r = (long)blockIdx.x * D;
    if (pk.splits > 0) {                                         // uniform
        for (int i = threadIdx.x; i < D; i += 256) d_o[r + i] = sum_splits(pk.parts, pk.splits, pk.stride, r + i);
    }
    float ss = 0.0f, dot = 0.0f;
    for (int i = threadIdx.x; i < D; i += 256) {
        const float xi = x[r + i];
        ss += xi * xi;
        dot += d_o[r + i] * w[i] * xi;
    }
    ss = block_sum<4>(ss, red);
    dot = block_sum<4>(dot, red);
    ss = ss / D + 1e-5f;
    const float inv = 1.0f / d_sqrtf(ss);
    const float cd = inv * inv * inv / (float)D * dot;
    if (threadIdx.x == 0) inv_out[blockIdx.x] = inv;
    // d_in == nullptr: the incoming residual gradient is zero (0 + v == v)
    for (int i = threadIdx.x; i < D; i += 256) {
        const float v = inv * d_o[r + i] * w[i] - cd * x[r + i];
        d_out[r + i] = d_in ? d_in[r + i] + v : v;
    }
}

// ── RMSNorm rows, one wave per row ──────────────────────────────────────
// The same two row kernels for D % 4 == 0 and D <= 256*NV: one wave per
// row (launched as one-wave blocks, so the rows spread over as many CUs as
// possible), lane l holding float4s l, 64 + l, ... of its row in
// registers, so every load of the row goes out together and the row sums
// are DPP reductions without block barriers.

// float4 i of row r of a split-K GEMM's output: sum_z parts[z] in z order,
// eight partial loads in flight at a time.
__device__ __forceinline__ float4 sum_splits4(const SplitK &pk, long i4) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 *p = reinterpret_cast<const float4 *>(pk.parts);
    const long st4 = pk.stride / 4;
    for (int z0 = 0; z0 < pk.splits; z0 += 8) {
        float4 pv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) pv[u] = p[(long)min(z0 + u, pk.splits - 1) * st4 + i4];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const bool in = z0 + u < pk.splits;
            v.x = in ? v.x + pv[u].x : v.x;
            v.y = in ? v.y + pv[u].y : v.y;
            v.z = in ? v.z + pv[u].z : v.z;
            v.w = in ? v.w + pv[u].w : v.w;
        }
    }
    return v;
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

// k_rmsnorm_rows, one wave per row (rmsnorm, pt_ops.c:5-12).
// With tok != nullptr the row is first gathered from the embedding table,
// in[row] = emb[tok[row]] (pt_train.c:189-191), and stored; rows < rows-1
// also mark their token in tok_bits.
template <int NV>
__global__ __launch_bounds__(256) void k_rmsnorm_rows_w(float *in, const float *w, float *out, int rows, int D,
                                                       SplitK pk, const float *cin, const int *tok, const float *emb,
                                                       unsigned *tok_bits) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * (int)(blockDim.x >> 6) + (threadIdx.x >> 6), d4 = D / 4;
    if (row >= rows) return;                                     // wave-uniform
    const long r4 = (long)row * d4;
    float4 *x4 = reinterpret_cast<float4 *>(in) + r4;
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 xv[NV], wv[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) wv[v] = w4[min(lane + 64 * v, d4 - 1)];
    if (tok) {                                                   // uniform
        const int tk = tok[row];
        if (lane == 0 && row < rows - 1) atomicOr(&tok_bits[tk >> 5], 1u << (tk & 31));
        const float4 *e4 = reinterpret_cast<const float4 *>(emb) + (long)tk * d4;
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const int c = min(lane + 64 * v, d4 - 1);
            xv[v] = e4[c];
            if (lane + 64 * v < d4) x4[c] = xv[v];
        }
    } else if (pk.splits > 0) {                                  // uniform
        const float4 *c4 = reinterpret_cast<const float4 *>(cin);
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const int c = min(lane + 64 * v, d4 - 1);
            xv[v] = sum_splits4(pk, r4 + c);
            if (cin) xv[v] = add4(c4[r4 + c], xv[v]);
            if (lane + 64 * v < d4) x4[c] = xv[v];
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; v++) xv[v] = x4[min(lane + 64 * v, d4 - 1)];
    }
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const float q = xv[v].x * xv[v].x + xv[v].y * xv[v].y + xv[v].z * xv[v].z + xv[v].w * xv[v].w;
        ss = lane + 64 * v < d4 ? ss + q : ss;
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / d_sqrtf(ss / D + 1e-5f);
    float4 *o4 = reinterpret_cast<float4 *>(out) + r4;
#pragma unroll
    for (int v = 0; v < NV; v++)
        if (lane + 64 * v < d4)
            o4[lane + 64 * v] = make_float4(xv[v].x * inv * wv[v].x, xv[v].y * inv * wv[v].y,
                                            xv[v].z * inv * wv[v].z, xv[v].w * inv * wv[v].w);
}

// k_rmsnorm_bwd_rows, one wave per row (pt_backward_ops.c:4-30).
template <int NV>
__global__ __launch_bounds__(256) void k_rmsnorm_bwd_rows_w(float *d_out, const float *d_in, float *d_o,
                                                           const float *x, const float *w, float *inv_out, int rows,
                                                           int D, SplitK pk) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * (int)(blockDim.x >> 6) + (threadIdx.x >> 6), d4 = D / 4;
    if (row >= rows) return;                                     // wave-uniform
    const long r4 = (long)row * d4;
    const float4 *x4 = reinterpret_cast<const float4 *>(x) + r4, *w4 = reinterpret_cast<const float4 *>(w);
    float4 *g4 = reinterpret_cast<float4 *>(d_o) + r4;
    float4 xv[NV], wv[NV], gv[NV], iv[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const int c = min(lane + 64 * v, d4 - 1);
        xv[v] = x4[c];
        wv[v] = w4[c];
        iv[v] = d_in ? reinterpret_cast<const float4 *>(d_in)[r4 + c] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (pk.splits > 0) {                                         // uniform
#pragma unroll
        for (int v = 0; v < NV; v++) {
            const int c = min(lane + 64 * v, d4 - 1);
            gv[v] = sum_splits4(pk, r4 + c);
            if (lane + 64 * v < d4) g4[c] = gv[v];
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; v++) gv[v] = g4[min(lane + 64 * v, d4 - 1)];
    }
    float ss = 0.0f, dot = 0.0f;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        const bool in = lane + 64 * v < d4;
        const float q = xv[v].x * xv[v].x + xv[v].y * xv[v].y + xv[v].z * xv[v].z + xv[v].w * xv[v].w;
        const float d = gv[v].x * wv[v].x * xv[v].x + gv[v].y * wv[v].y * xv[v].y + gv[v].z * wv[v].z * xv[v].z +
                        gv[v].w * wv[v].w * xv[v].w;
        ss = in ? ss + q : ss;
        dot = in ? dot + d : dot;
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    ss = ss / D + 1e-5f;
    const float inv = 1.0f / d_sqrtf(ss);
    const float cd = inv * inv * inv / (float)D * dot;
    if (lane == 0) inv_out[row] = inv;
    float4 *o4 = reinterpret_cast<float4 *>(d_out) + r4;
#pragma unroll
    for (int v = 0; v < NV; v++) {
        if (lane + 64 * v < d4) {
            float4 o;
            o.x = iv[v].x + (inv * gv[v].x * wv[v].x - cd * xv[v].x);
            o.y = iv[v].y + (inv * gv[v].y * wv[v].y - cd * xv[v].y);
            o.z = iv[v].z + (inv * gv[v].z * wv[v].z - cd * xv[v].z);
            o.w = iv[v].w + (inv * gv[v].w * wv[v].w - cd * xv[v].w);
            o4[lane + 64 * v] = o;
        }
    }
}

// The d_w half of every RMSNorm of the step in one launch: for norm
// j = blockIdx.x / cb, d_w[i] = sum_t d_o[t][i]*x[t][i]*inv[t] (written: each
// norm weight is used once per step); 64 columns per block, 16 interleaved
// row slices summed in LDS.
// With the weight's SGD step (pt_train.c:870-873): w[i] -= lr * d_w[i].
struct NormDw {
    float *d_w;
    const float *d_o, *x, *inv;
    float *w;
};
__device__ __forceinline__ void rmsnorm_dw_block(const NormDw *nd, int cb, int R, int D, int b, float lr) {
    __shared__ float part[16][64];
    const NormDw e = nd[b / cb];
    const int c = threadIdx.x & 63, sl = threadIdx.x >> 6;
    const int i = (b % cb) * 64 + c;
    float acc = 0.0f;
    if (i < D) {
#pragma unroll 4
        for (int t = sl; t < R; t += 16) acc += e.d_o[(long)t * D + i] * e.x[(long)t * D + i] * e.inv[t];
    }
    part[sl][c] = acc;
    __syncthreads();
    if (sl == 0 && i < D) {
        float g = 0.0f;
        for (int k = 0; k < 16; k++) g += part[k][c];
        e.d_w[i] = g;
        e.w[i] -= lr * g;
    }
}

// Attention backward, row half (pt_train.c:780-811): for (t < R, head h):
// d_att_s, the softmax backward dot, ds = d_pre*scale (kept for the column
// half) and d_q[t] = sum_t2 ds[t2] k[t2].  Dynamic LDS: das[T].
template <int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn_bwd_rows(const float *qkv, const float *att,
                                                                const float *d_aout, float *ds, float *d_q, int T,
                                                                int D, int QS, int KV, int hd, int kv_mul,
                                                                float scale) {
    extern __shared__ float das[];
    __shared__ float part[kAttnPart];
    __shared__ float red[4];
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, hd4 = hd >> 2, sub = tid % G;
    const float *arow = att + ((long)h * T + t) * T;
    const int ko = D + (h / kv_mul) * hd, vo = D + KV + (h / kv_mul) * hd;
    const float4 g4 = sub < hd4 ? reinterpret_cast<const float4 *>(d_aout + (long)t * D + h * hd)[sub]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
    const int n = t + 1;
    row_dots<G>(qkv + vo, QS, g4, hd4, n, das, 1.0f);
    __syncthreads();
    float dot = 0.0f;
    for (int t2 = tid; t2 < n; t2 += kAttnThreads) dot += das[t2] * arow[t2];
    dot = block_sum<4>(dot, red);
    float *dsrow = ds + ((long)h * T + t) * T;
    for (int t2 = tid; t2 < n; t2 += kAttnThreads) {
        const float d = arow[t2] * (das[t2] - dot) * scale;
        das[t2] = d;
        dsrow[t2] = d;
    }
    __syncthreads();
    const float o = weighted_rows<G>(qkv + ko, QS, das, hd4, n, part);
    if (tid < hd) d_q[(long)t * D + h * hd + tid] = o;
}

// Attention backward, column half: for (t2 < R, head h):
// d_v[t2] = sum_{t>=t2} att[t][t2] d_aout[t],  d_k[t2] = sum_{t>=t2} ds[t][t2] q[t].
// Dynamic LDS: w[2*T].
template <int G>
__global__ __launch_bounds__(kAttnThreads) void k_attn_bwd_cols(const float *qkv, const float *att, const float *ds,
                                                                const float *d_aout, float *d_k, float *d_v, int T,
                                                                int R, int D, int QS, int KV, int hd, int kv_mul) {
    extern __shared__ float sm[];
    __shared__ float part[kAttnPart];
    float *wa = sm, *wd = sm + T;
    const int t2 = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, hd4 = hd >> 2;
    const int kvo = (h / kv_mul) * hd, n = R - t2;
    for (int k = tid; k < n; k += kAttnThreads) {
        const long a = ((long)h * T + t2 + k) * T + t2;
        wa[k] = att[a];
        wd[k] = ds[a];
    }
    __syncthreads();
    const float dv = weighted_rows<G>(d_aout + (long)t2 * D + h * hd, D, wa, hd4, n, part);
    const float dk = weighted_rows<G>(qkv + (long)t2 * QS + h * hd, QS, wd, hd4, n, part);
    if (tid < hd) {
        d_v[(long)t2 * KV + kvo + tid] = dv;
        d_k[(long)t2 * KV + kvo + tid] = dk;
    }
}

// ── attention on the matrix cores ────────────────────────────────────────
// The same three attention kernels for head_dim = 16*HQ (HQ <= 8), with
// n_kv_heads == n_heads (training requires it), on v_mfma_f32_16x16x4_f32.
// One block of kMW waves per (16-row tile, head).  Lane l supplies
// A[l%16][l/16] and B[l/16][l%16]; result register r of lane l is
// C[4*(l/16)+r][l%16].  A and B may share any order of the contraction
// index: over head_dim, lane group g = l/16 takes the quarter
// [4*HQ*g, 4*HQ*(g+1)) as HQ float4s (step 4q+c uses component c of float4
// q); over positions, step s of a 16-position block takes position 4g + s,
// so a lane's four weights are one float4 in LDS.  Sums therefore run in a
// different order from the reference's sequential loops.
constexpr int kMW = 8, kMT = 64 * kMW;
// Rows per block of the forward and row-backward kernels.  Their MFMA tiles
// still span 16 rows (the 8 rows after the block's own are computed and
// dropped), but each wave's per-row softmax work covers one row instead of
// two.  The slowest block (the last rows, every key) sets the launch time,
// so halving its softmax share pays for the doubled MFMA work: step 0.808-
// 0.813 -> 0.790-0.797 ms (stories15M T=256, same-box A/B).
constexpr int kAttnRows = 8;
static_assert(kAttnRows % kMW == 0 && kAttnRows <= 16, "rows per wave");

typedef float f4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4v mfma4(float a, float b, f4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// rope_backward (pt_backward_ops.c:52-69) of element c of a head's column
// pair at position t, given its pair partner: o[i] = g0*c + g1*s,
// o[i+1] = -g0*s + g1*c for the pair (g0, g1) = (col 2k, col 2k+1).
__device__ __forceinline__ float rope_bwd_elem(float v, float pv, int col, int hd, int t) {
    float cs, sn;
    d_rope_cs(col & ~1, hd, t, &cs, &sn);
    return (col & 1) ? -pv * sn + v * cs : v * cs + pv * sn;
}

// sc[i][16*kb + j] = mul * (a[r0+i] . b[16*kb+j]) over head_dim for this
// wave's key blocks kb = wave, wave + kMW, ... < nkb (LDS rows of `pitch`
// floats).  Rows past a_rows / b_rows read the operand's last row; those
// entries are never used.
template <int HQ>
__device__ __forceinline__ void attn_dots(const float *a, long lda, int r0, int a_rows, const float *b, long ldb,
                                          int b_rows, int nkb, float mul, float *sc, int pitch) {
    constexpr int U = HQ <= 3 ? 2 : 1;                 // key blocks in flight per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
    float4 av[HQ];
    const float4 *ap = reinterpret_cast<const float4 *>(a + (long)min(r0 + li, a_rows - 1) * lda) + g * HQ;
#pragma unroll
    for (int q = 0; q < HQ; q++) av[q] = ap[q];
    for (int kb0 = wave; kb0 < nkb; kb0 += U * kMW) {
        float4 bv[U][HQ];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int key = min((kb0 + u * kMW) * 16 + li, b_rows - 1);
            const float4 *bp = reinterpret_cast<const float4 *>(b + (long)key * ldb) + g * HQ;
#pragma unroll
            for (int q = 0; q < HQ; q++) bv[u][q] = bp[q];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int kb = kb0 + u * kMW;
            f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q = 0; q < HQ; q++) {
                acc = mfma4(av[q].x, bv[u][q].x, acc);
                acc = mfma4(av[q].y, bv[u][q].y, acc);
                acc = mfma4(av[q].z, bv[u][q].z, acc);
                acc = mfma4(av[q].w, bv[u][q].w, acc);
            }
            if (kb < nkb) {                                 // uniform
#pragma unroll
                for (int r = 0; r < 4; r++) sc[(4 * g + r) * pitch + kb * 16 + li] = acc[r] * mul;
            }
        }
    }
}

// acc[cb] = this wave's share of sum_key sc[i][key] * v[key][16*cb + j]
// over its key blocks (the weights in LDS rows of `pitch` floats).  load()
// fetches the operand rows of the wave's first U key blocks and may be
// issued before the weights are ready; run() fetches any further ones.
template <int HQ>
struct AttnWsum {
    static constexpr int U = HQ <= 3 ? 2 : 1;
    float vv[U][4][HQ];
    __device__ __forceinline__ void load(const float *v, long ldv, int v_rows, int kb0) {
        const int lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int key = min((kb0 + u * kMW) * 16 + 4 * g + s, v_rows - 1);
#pragma unroll
                for (int cb = 0; cb < HQ; cb++) vv[u][s][cb] = v[(long)key * ldv + cb * 16 + li];
            }
    }
    __device__ __forceinline__ void run(const float *sc, int pitch, const float *v, long ldv, int v_rows, int nkb,
                                        f4v (&acc)[HQ]) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
#pragma unroll
        for (int cb = 0; cb < HQ; cb++) acc[cb] = f4v{0.f, 0.f, 0.f, 0.f};
        for (int kb0 = wave; kb0 < nkb; kb0 += U * kMW) {
            if (kb0 != wave) load(v, ldv, v_rows, kb0);     // uniform
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int kb = kb0 + u * kMW;
                if (kb < nkb) {                             // uniform
                    const float4 w = *reinterpret_cast<const float4 *>(sc + li * pitch + kb * 16 + 4 * g);
#pragma unroll
                    for (int cb = 0; cb < HQ; cb++) {
                        acc[cb] = mfma4(w.x, vv[u][0][cb], acc[cb]);
                        acc[cb] = mfma4(w.y, vv[u][1][cb], acc[cb]);
                        acc[cb] = mfma4(w.z, vv[u][2][cb], acc[cb]);
                        acc[cb] = mfma4(w.w, vv[u][3][cb], acc[cb]);
                    }
                }
            }
        }
    }
};

// A row's first kw (a multiple of 16) LDS entries, 4 consecutive per lane
// in up to kAttnChunks chunks of 256 (T <= 1024): x[c] holds keys
// 256c + 4*lane + (0..3); chunks at or past kw read as zeros.  Addresses
// are clamped into the row so that every lane's read stays inside it.
constexpr int kAttnChunks = 4;
__device__ __forceinline__ void row_chunks(const float *row, int kw, float4 (&x)[kAttnChunks]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int c = 0; c < kAttnChunks; c++) {
        x[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (256 * c < kw) x[c] = *reinterpret_cast<const float4 *>(row + min(256 * c + 4 * lane, kw - 4));
    }
}

// Sums the kMW waves' 16 x 16*HQ tiles in wave order through LDS `red`
// (kMW*16*16*HQ floats) and hands each element to out(i, c, value, pair),
// pair being element (i, c^1): columns c and c^1 sit in lanes l and l^1
// (16*HQ and kMT are even), and every pass over e has whole waves active
// (16*16*HQ is a multiple of 64), so a DPP swap reads it.
template <int HQ, typename F>
__device__ __forceinline__ void attn_reduce(const f4v (&acc)[HQ], float *red, F &&out) {
    constexpr int HD = 16 * HQ;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, li = lane & 15, g = lane >> 4;
    __syncthreads();                                       // earlier readers of red are done
#pragma unroll
    for (int cb = 0; cb < HQ; cb++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[(wave * 16 + 4 * g + r) * HD + cb * 16 + li] = acc[cb][r];
    __syncthreads();
    for (int e = threadIdx.x; e < 16 * HD; e += kMT) {
        float v = red[e];
#pragma unroll
        for (int w = 1; w < kMW; w++) v += red[w * 16 * HD + e];
        out(e / HD, e % HD, v, dpp_xor1(v));
    }
}

// Causal attention forward (pt_train.c:224-255) for positions
// [RT*blockIdx.x, +RT) of head blockIdx.y (RT = kAttnRows; the 16-row MFMA
// tiles also cover the next 16 - RT rows, whose results are dropped):
// scores into LDS, a softmax per
// row (one wave per row; max, then e^(s - max) and its sum, then the 1/sum
// scaling, as the reference), the probabilities to att (zeros past the
// diagonal), then att_out = P.V.  Dynamic LDS: max(16*pitch, kMW*16*hd)
// floats, pitch = 16*ceil(T/16) + 4.
template <int HQ>
__global__ __launch_bounds__(kMT) void k_attn_fwd_mfma(const float *qkv, float *att, float *att_out, int T, int D,
                                                      int QS, float scale, int pitch) {
    extern __shared__ float lds[];
    constexpr int HD = 16 * HQ;
    constexpr int RT = kAttnRows;
    const int r0 = blockIdx.x * RT, h = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nkb = (min(r0 + RT, T) + 15) / 16, kw = nkb * 16;
    const float *q = qkv + h * HD, *k = qkv + D + h * HD, *v = qkv + 2 * D + h * HD;
    attn_dots<HQ>(q, QS, r0, T, k, QS, T, nkb, scale, lds, pitch);
    AttnWsum<HQ> ws;
    ws.load(v, QS, T, wave);                                // in flight during the softmax
    __syncthreads();
    // the wave's rows i = wave + w*kMW, in lockstep (rows past T compute
    // unused values and store nothing)
    constexpr int RW = RT / kMW;
    float4 x[RW][kAttnChunks];
    float mx[RW], sum[RW];
#pragma unroll
    for (int w = 0; w < RW; w++) {
        const int n = r0 + wave + w * kMW + 1;
        row_chunks(lds + (wave + w * kMW) * pitch, kw, x[w]);
        mx[w] = -INFINITY;
#pragma unroll
        for (int c = 0; c < kAttnChunks; c++) {
            const int j = 256 * c + 4 * lane;
#pragma unroll
            for (int e = 0; e < 4; e++) mx[w] = j + e < n ? fmaxf(mx[w], (&x[w][c].x)[e]) : mx[w];
        }
    }
#pragma unroll
    for (int w = 0; w < RW; w++) mx[w] = wave_max(mx[w]);
#pragma unroll
    for (int w = 0; w < RW; w++) {
        const int n = r0 + wave + w * kMW + 1;
        sum[w] = 0.0f;
#pragma unroll
        for (int c = 0; c < kAttnChunks; c++) {
            if (256 * c < kw) {                             // uniform
                const int j = 256 * c + 4 * lane;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float ex = j + e < n ? d_expf((&x[w][c].x)[e] - mx[w]) : 0.0f;
                    (&x[w][c].x)[e] = ex;
                    sum[w] += ex;
                }
            }
        }
    }
#pragma unroll
    for (int w = 0; w < RW; w++) sum[w] = wave_sum(sum[w]);
#pragma unroll
    for (int w = 0; w < RW; w++) {
        const int i = wave + w * kMW, t = r0 + i;
        if (t >= T) continue;                               // uniform
        const float inv = 1.0f / sum[w];
        float *row = lds + i * pitch, *arow = att + ((long)h * T + t) * T;
#pragma unroll
        for (int c = 0; c < kAttnChunks; c++) {
            const int j = 256 * c + 4 * lane;
            const float4 a = make_float4(x[w][c].x * inv, x[w][c].y * inv, x[w][c].z * inv, x[w][c].w * inv);
            if (j < kw) *reinterpret_cast<float4 *>(row + j) = a;
            if ((T & 3) == 0) {
                if (j < T) *reinterpret_cast<float4 *>(arow + j) = a;
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (j + e < T) arow[j + e] = (&a.x)[e];
            }
        }
    }
    __syncthreads();
    f4v acc[HQ];
    ws.run(lds, pitch, v, QS, T, nkb, acc);
    attn_reduce<HQ>(acc, lds, [&](int i, int c, float o, float) {
        if (i < RT && r0 + i < T) att_out[(long)(r0 + i) * D + h * HD + c] = o;
    });
}

// Attention backward, row half (pt_train.c:780-811) for rows t < R in
// [RT*blockIdx.x, +RT) of head blockIdx.y (RT = kAttnRows, 16-row MFMA tiles
// as in the forward; the extra rows' d_aout is read back as another block
// leaves it and only feeds dropped results): d_att = d_aout.V^T into LDS, per
// row the softmax backward dot and ds = att*(d_att - dot)*scale (kept for
// the column half), then d_q = ds.K, stored after rope_backward into the q
// columns of the fused [dq | dk | dv] row d_qkv.  LDS as k_attn_fwd_mfma.
template <int HQ>
// With d_res non-null (D a multiple of 4*kMW), the block first computes its
// own tile of d_aout = d_res . Wo (backward_input of the Wo projection,
// pt_train.c:729-730: rows [r0, r0+RT), head h's columns), each wave over
// a D/kMW slice of the contraction summed in wave order, and writes it for
// the column kernel; the first dot product below reads it back.
__global__ __launch_bounds__(kMT) void k_attn_bwd_rows_mfma(const float *qkv, const float *att, float *d_aout,
                                                           const float *d_res, const float *wo, float *ds,
                                                           float *d_qkv, int T, int R, int D, int QS, float scale,
                                                           int pitch) {
    extern __shared__ float lds[];
    constexpr int RT = kAttnRows, HD = 16 * HQ, RW = RT / kMW;   // rows per wave
    const int r0 = blockIdx.x * RT, h = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nkb = (min(r0 + RT, R) + 15) / 16, kw = nkb * 16;
    const float *k = qkv + D + h * HD, *v = qkv + 2 * D + h * HD;
    if (d_res) {                                            // uniform
        const int li = lane & 15, g = lane >> 4, ks = D / kMW, k0 = wave * ks;
        const float *ap = d_res + (long)min(r0 + li, R - 1) * D + k0 + g;
        const float *bp = wo + (long)(k0 + g) * D + h * HD + li;
        f4v acc[HQ];
#pragma unroll
        for (int cb = 0; cb < HQ; cb++) acc[cb] = f4v{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < ks; s += 4) {
            const float a = ap[s];
#pragma unroll
            for (int cb = 0; cb < HQ; cb++) acc[cb] = mfma4(a, bp[(long)s * D + cb * 16], acc[cb]);
        }
        attn_reduce<HQ>(acc, lds, [&](int i, int c, float o, float) {
            if (i < RT && r0 + i < R) d_aout[(long)(r0 + i) * D + h * HD + c] = o;
        });
        __syncthreads();                                   // the tile is written; lds is free again
    }
    // this wave's att rows (keys < n, clamped), fetched with the GEMM operands
    float ar[RW][kAttnChunks][4];
#pragma unroll
    for (int w = 0; w < RW; w++) {
        const int t = min(r0 + wave + w * kMW, R - 1);
        const float *arow = att + ((long)h * T + t) * T;
#pragma unroll
        for (int c = 0; c < kAttnChunks; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) ar[w][c][e] = 256 * c < kw ? arow[min(256 * c + 4 * lane + e, t)] : 0.0f;
    }
    attn_dots<HQ>(d_aout + h * HD, D, r0, R, v, QS, T, nkb, 1.0f, lds, pitch);
    AttnWsum<HQ> ws;
    ws.load(k, QS, T, wave);
    __syncthreads();
    // the wave's rows i = wave + w*kMW in lockstep, as in the forward
    float4 x[RW][kAttnChunks];
    float dot[RW];
#pragma unroll
    for (int w = 0; w < RW; w++) {
        const int n = r0 + wave + w * kMW + 1;
        row_chunks(lds + (wave + w * kMW) * pitch, kw, x[w]);
        dot[w] = 0.0f;
#pragma unroll
        for (int c = 0; c < kAttnChunks; c++) {
            const int j = 256 * c + 4 * lane;
#pragma unroll
            for (int e = 0; e < 4; e++) dot[w] = j + e < n ? dot[w] + (&x[w][c].x)[e] * ar[w][c][e] : dot[w];
        }
    }
#pragma unroll
    for (int w = 0; w < RW; w++) dot[w] = wave_sum(dot[w]);
#pragma unroll
    for (int w = 0; w < RW; w++) {
        const int i = wave + w * kMW, t = r0 + i;
        if (t >= R) continue;                               // uniform
        const int n = t + 1;
        float *row = lds + i * pitch, *dsrow = ds + ((long)h * T + t) * T;
#pragma unroll
        for (int c = 0; c < kAttnChunks; c++) {
            if (256 * c < kw) {                             // uniform
                const int j = 256 * c + 4 * lane;
                float4 d;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const bool in = j + e < n;
                    (&d.x)[e] = in ? ar[w][c][e] * ((&x[w][c].x)[e] - dot[w]) * scale : 0.0f;
                    if (in) dsrow[j + e] = (&d.x)[e];
                }
                if (j < kw) *reinterpret_cast<float4 *>(row + j) = d;
            }
        }
    }
    __syncthreads();
    f4v acc[HQ];
    ws.run(lds, pitch, k, QS, T, nkb, acc);
    attn_reduce<HQ>(acc, lds, [&](int i, int c, float o, float po) {
        const int t = r0 + i;
        if (i < RT && t < R) d_qkv[(long)t * QS + h * HD + c] = rope_bwd_elem(o, po, h * HD + c, HD, t);
    });
}

// Attention backward, column half, for keys t2 < R in [16*blockIdx.x, +16)
// of head blockIdx.y: d_v[t2] = sum_{t2<=t<R} att[t][t2] d_aout[t] and
// d_k[t2] = sum_{t2<=t<R} ds[t][t2] q[t], stored into the v and (after
// rope_backward) k columns of d_qkv.  ds holds only t2 <= t, so the weights
// are selected (never multiplied) by that condition.  Dynamic LDS:
// kMW*16*hd floats.
template <int HQ>
__global__ __launch_bounds__(kMT) void k_attn_bwd_cols_mfma(const float *qkv, const float *att, const float *ds,
                                                           const float *d_aout, float *d_qkv, int T, int R, int D,
                                                           int QS) {
    extern __shared__ float lds[];
    constexpr int HD = 16 * HQ, U = HQ <= 3 ? 2 : 1;
    const int k0 = blockIdx.x * 16, h = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane & 15, g = lane >> 4, ntb = (R + 15) / 16;
    const int key = min(k0 + li, T - 1);
    const float *q = qkv + h * HD, *go = d_aout + h * HD;
    const float *ah = att + (long)h * T * T + key, *dh = ds + (long)h * T * T + key;
    f4v av[HQ], ak[HQ];
#pragma unroll
    for (int cb = 0; cb < HQ; cb++) av[cb] = ak[cb] = f4v{0.f, 0.f, 0.f, 0.f};
    for (int tb0 = blockIdx.x + wave; tb0 < ntb; tb0 += U * kMW) {
        float wa[U][4], wd[U][4], bo[U][4][HQ], bq[U][4][HQ];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int t = min((tb0 + u * kMW) * 16 + 4 * g + s, R - 1);
                wa[u][s] = ah[(long)t * T];
                wd[u][s] = dh[(long)t * T];
#pragma unroll
                for (int cb = 0; cb < HQ; cb++) {
                    bo[u][s][cb] = go[(long)t * D + cb * 16 + li];
                    bq[u][s][cb] = q[(long)t * QS + cb * 16 + li];
                }
            }
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const int t = (tb0 + u * kMW) * 16 + 4 * g + s;
                const bool use = t < R && t >= k0 + li;
                const float a1 = use ? wa[u][s] : 0.0f, a2 = use ? wd[u][s] : 0.0f;
#pragma unroll
                for (int cb = 0; cb < HQ; cb++) {
                    av[cb] = mfma4(a1, bo[u][s][cb], av[cb]);
                    ak[cb] = mfma4(a2, bq[u][s][cb], ak[cb]);
                }
            }
    }
    attn_reduce<HQ>(av, lds, [&](int i, int c, float o, float) {
        if (k0 + i < R) d_qkv[(long)(k0 + i) * QS + 2 * D + h * HD + c] = o;
    });
    attn_reduce<HQ>(ak, lds, [&](int i, int c, float o, float po) {
        const int t = k0 + i;
        if (t < R) d_qkv[(long)t * QS + D + h * HD + c] = rope_bwd_elem(o, po, h * HD + c, HD, t);
    });
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

// embedding_backward (pt_backward_ops.c:90-95) in the reference's order:
// the block of the first position holding a token accumulates, per column,
// every position with that token in ascending t.  One pass over tok marks
// the block's positions in an LDS bit mask (any earlier one hands the token
// to an earlier block); each column then walks the mask in ascending order.
// The owner block then applies the row's SGD step (pt_train.c:870-873) and
// clears the token's bit in tok_bits.  pmask: (R + 31) / 32 words of LDS.
__device__ __forceinline__ void embed_bwd_block(const int *tok, const float *d_res, float *g_emb, float *w_emb,
                                                unsigned *tok_bits, float lr, int R, int D, int t, unsigned *pmask) {
    const int nw = (R + 31) / 32, tk = tok[t];
    for (int w = threadIdx.x; w < nw; w += blockDim.x) pmask[w] = 0u;
    __syncthreads();
    int earlier = 0;
    for (int k = threadIdx.x; k < R; k += blockDim.x) {
        if (tok[k] == tk) {
            if (k < t) earlier = 1;
            else atomicOr(&pmask[k >> 5], 1u << (k & 31));
        }
    }
    if (__syncthreads_or(earlier)) return;          // uniform: an earlier block owns this token
    for (int j = threadIdx.x; j < D; j += blockDim.x) {
        float acc = g_emb[(long)tk * D + j];
        for (int w = 0; w < nw; w++) {
            for (unsigned bits = pmask[w]; bits; bits &= bits - 1)
                acc += d_res[(long)(32 * w + __builtin_ctz(bits)) * D + j];
        }
        g_emb[(long)tk * D + j] = acc;
        w_emb[(long)tk * D + j] -= lr * acc;
    }
    if (threadIdx.x == 0) atomicAnd(&tok_bits[tk >> 5], ~(1u << (tk & 31)));
}

// The step's last reductions and updates, one launch of 1024-thread blocks:
// blocks [0, nn) the RMSNorm dW columns with their SGD steps, [nn, nn + R)
// the embedding backward (and SGD step) of position b - nn's token, and
// block nn + R the mean loss.  Dynamic LDS: the embedding backward's
// (R + 31) / 32 mask words.
__global__ __launch_bounds__(1024) void k_step_tail(const NormDw *nd, int cb, int nn, int R, int D, const int *tok,
                                                    const float *d_res, float *g_emb, float *w_emb,
                                                    unsigned *tok_bits, const float *lr, const float *row_loss,
                                                    float *loss) {
    extern __shared__ unsigned pmask[];
    const int b = blockIdx.x;
    const float lrv = *lr;
    if (b < nn) rmsnorm_dw_block(nd, cb, R, D, b, lrv);
    else if (b < nn + R) embed_bwd_block(tok, d_res, g_emb, w_emb, tok_bits, lrv, R, D, b - nn, pmask);
    else loss_mean_block<16>(row_loss, R, loss);
}

// One wave of dependent FMAs for a fixed count (several ms): it holds the
// stream while the host enqueues a traced step behind it.  The store is
// never taken; it keeps the loop live.
constexpr int kHoldIters = 1 << 20;
__global__ void k_hold(float *sink, int iters) {
    float v = (float)threadIdx.x;
    for (int i = 0; i < iters; i++) v = fmaf(v, 0.999f, 1.0f);
    if (v == -1.0f) *sink = v;
}

// Zero fill (pt_zero_grads, pt_train.c:425-427), a kernel rather than a
// memset node so the step can be captured.
__global__ void k_fill0(float *p, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.0f;
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
        (2 * L + 2) * T * D, (2 * L + 1) * T * D, T * H, L * T * 2 * H, L * T * H, T * D, T * D, T * KV, T * KV,
        L * T * QS, NH * T * T, (2 * L + 1) * T, T, 64, ts->ws_floats, T, 1,
        (gemm_group_desc_bytes(4 * (int)L + 1) + 3) / 4, (sizeof(NormDw) * (2 * L + 1) + 3) / 4, (V + 31) / 32};
    float *dw_desc = nullptr;
    float **dst[] = {&ts->res, &ts->res_att, &ts->xb_att, &ts->qkv, &ts->att, &ts->att_out, &ts->xb_ffn, &ts->h13,
                     &ts->sh, &ts->x_final, &ts->logits, &ts->gmem, &ts->d_res, &ts->d_xb, &ts->d_sh, &ts->d_h13,
                     &ts->shb, &ts->d_aout, &ts->d_q, &ts->d_k, &ts->d_v, &ts->d_qkv, &ts->ds, &ts->row_inv,
                     &ts->row_loss, &ts->loss, &ts->ws, (float **)&ts->tok, &ts->lr, &dw_desc, &ts->nd_desc,
                     (float **)&ts->tok_bits};
    const int nbuf = (int)(sizeof(sizes) / sizeof(sizes[0]));
    size_t total = 0;
    for (int i = 0; i < nbuf; i++) total += align_up(sizes[i], 64);
    hipError_t e = hipMalloc(&ts->mem, total * sizeof(float));
    if (e != hipSuccess) { delete ts; return hip_check(e, "hipMalloc(training state)"); }
    size_t o = 0;
    for (int i = 0; i < nbuf; i++) { *dst[i] = ts->mem + o; o += align_up(sizes[i], 64); }
    ts->dw_desc = dw_desc;
    e = hipMemsetAsync(ts->mem, 0, total * sizeof(float), lib_stream());
    if (e == hipSuccess) e = hipStreamSynchronize(lib_stream());
    if (e != hipSuccess) { (void)hipFree(ts->mem); delete ts; return hip_check(e, "zero training state"); }
    ts->lr_off = ts->lr - reinterpret_cast<float *>(ts->tok);
    e = hipHostMalloc(reinterpret_cast<void **>(&ts->pin), (size_t)(ts->lr_off + 2) * sizeof(float), hipHostMallocDefault);
    if (e != hipSuccess) { (void)hipFree(ts->mem); delete ts; return hip_check(e, "hipHostMalloc(training staging)"); }
    const char *eager = getenv("PTMI_TRAIN_EAGER");
    ts->eager = eager && eager[0] == '1';
    const char *fuse = getenv("PTMI_TRAIN_FUSE_NORM");
    if (fuse) ts->fuse_norm = atoi(fuse) & 7;
    m->train = ts;
    return PTMI_OK;
}

void train_destroy(ptmi_model *m) {
    if (!m->train) return;
    if (m->train->exec) (void)hipGraphExecDestroy(m->train->exec);
    if (m->train->graph) (void)hipGraphDestroy(m->train->graph);
    (void)hipFree(m->train->mem);
    (void)hipHostFree(m->train->pin);
    delete m->train;
    m->train = nullptr;
}

namespace {

int gemm(hipStream_t s, TrainState *ts, int op, const float *A, long lda, const float *B, long ldb, float *C, long ldc,
         int M, int N, int K, int acc, const float *Cin = nullptr, SplitK *defer = nullptr,
         const GemmEpi *epi = nullptr, const GemmNorm *norm = nullptr) {
    return launch_gemm(op, A, lda, B, ldb, C, ldc, M, N, K, acc, ts->ws, ts->ws_floats, s, Cin, defer, epi, norm);
}

void fill0(hipStream_t s, float *p, long n) {
    hipLaunchKernelGGL(k_fill0, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
}

// Descriptor tables of the grouped weight-gradient launches for this T:
// per layer dW2 += d_res^T sh, dW13 += d_h13^T x_ffn, dWo += d_res^T att_out,
// dWqkv += d_qkv^T x_att, plus the classifier's dWcls += d_logits^T x_final;
// and the 2L+1 RMSNorm dW reductions, in the d_res version order the dX
// chain produces (final norm, then per layer from the last: ffn, att).
int train_descriptors(ptmi_model *m, int T) {
    TrainState *ts = m->train;
    if (ts->desc_T == T) return PTMI_OK;
    const Resident *r = m->res;
    const Config &c = m->c;
    const int D = c.dim, H = c.hidden, L = c.n_layers, V = c.vocab, KV = c.kv_dim, QS = D + 2 * KV, R = T - 1;
    const long TD = (long)T * D;
    auto G = [&](const float *p) { return ts->gmem + (p - r->mem); };
    auto W = [&](const float *p) { return r->mem + (p - r->mem); };     // the weight, writable (SGD)
    auto dres = [&](int k) { return ts->d_res + (long)k * TD; };
    auto dxb = [&](int k) { return ts->d_xb + (long)k * TD; };
    // Every weight's SGD step (pt_sgd_update, pt_train.c:870-896) is fused
    // into the kernel that writes its gradient: the dW GEMMs' epilogues, the
    // RMSNorm dW reductions, and, for the embedding rows of this step's
    // tokens, the embedding backward.  A classifier tied to the embedding
    // leaves those rows (bits of tok_bits) to the embedding backward.
    const bool tied = r->wcls == r->emb;
    std::vector<TnGemm> g;
    std::vector<NormDw> nd;
    g.push_back({ts->logits, V, ts->x_final, D, G(r->wcls), D, V, D, R, W(r->wcls), tied ? ts->tok_bits : nullptr});
    nd.push_back({G(r->rms_final), dxb(0), ts->res + L * TD, ts->row_inv, W(r->rms_final)});
    int v = 1;
    for (int l = L - 1; l >= 0; l--) {
        const float *xa = ts->xb_att + l * TD, *xf = ts->xb_ffn + l * TD, *ao = ts->att_out + l * TD;
        const float *rin = ts->res + l * TD, *rmid = ts->res_att + l * TD;
        const float *w2 = r->w2 + (long)l * D * H, *w13 = r->w13 + (long)l * 2 * H * D;
        const float *wo = r->wo + (long)l * D * D, *wqkv = r->wqkv + (long)l * QS * D;
        const float *dh13 = ts->d_h13 + (long)l * T * 2 * H, *shb = ts->shb + (long)l * T * H;
        const float *dqkv = ts->d_qkv + (long)l * T * QS;
        g.push_back({dres(v), D, shb, H, G(w2), H, D, H, R, W(w2)});            // FFN reads d_res[v]
        g.push_back({dh13, 2 * H, xf, D, G(w13), D, 2 * H, D, R, W(w13)});
        nd.push_back({G(r->rms_ffn + (long)l * D), dxb(v), rmid, ts->row_inv + (long)v * T, W(r->rms_ffn + (long)l * D)});
        v++;
        g.push_back({dres(v), D, ao, D, G(wo), D, D, D, R, W(wo)});             // Wo reads d_res[v+1]
        g.push_back({dqkv, QS, xa, D, G(wqkv), D, QS, D, R, W(wqkv)});
        nd.push_back({G(r->rms_att + (long)l * D), dxb(v), rin, ts->row_inv + (long)v * T, W(r->rms_att + (long)l * D)});
        v++;
    }
    std::vector<char> host(gemm_group_desc_bytes((int)g.size()));
    int tiles = 0, vec = 0, st;
    if ((st = gemm_tn_group_prepare(g.data(), (int)g.size(), ts->lr, host.data(), &tiles, &vec))) return st;
    PTMI_HIP(hipMemcpy(ts->dw_desc, host.data(), host.size(), hipMemcpyHostToDevice));
    PTMI_HIP(hipMemcpy(ts->nd_desc, nd.data(), nd.size() * sizeof(NormDw), hipMemcpyHostToDevice));
    ts->n_dw = (int)g.size();
    ts->dw_tiles = tiles;
    ts->dw_cls_tiles = ((V + 31) / 32) * ((D + 31) / 32);
    ts->dw_vec = vec;
    ts->desc_T = T;
    return PTMI_OK;
}

// The whole step on stream s; T fixed, tokens and lr read from device
// memory (ts->tok, ts->lr), so it can be captured once per T.
// Device-timed spans of one training step, for the reference's trace
// (pitorch/profiler/trace.c): begin/end record HIP events on the step's
// stream around the launches of a phase, nested like pt_train.c's
// pt_trace_begin/pt_trace_end calls; spans are kept in the order they end,
// as trace.c records them.
struct TrainTracer {
    struct Rec { const char *name, *cat; int layer, depth; hipEvent_t b, e; };
    std::vector<Rec> open, done;
    hipStream_t s;
    int begin(const char *name, const char *cat, int layer) {
        Rec r = {name, cat, layer, (int)open.size(), nullptr, nullptr};
        PTMI_HIP(hipEventCreate(&r.b));
        PTMI_HIP(hipEventCreate(&r.e));
        PTMI_HIP(hipEventRecord(r.b, s));
        open.push_back(r);
        return PTMI_OK;
    }
    int end() {
        if (open.empty()) return set_error(PTMI_ERR_STATE, "trace span end without begin");
        Rec r = open.back();
        open.pop_back();
        PTMI_HIP(hipEventRecord(r.e, s));
        done.push_back(r);
        return PTMI_OK;
    }
    void release() {
        for (Rec &r : open) { (void)hipEventDestroy(r.b); (void)hipEventDestroy(r.e); }
        for (Rec &r : done) { (void)hipEventDestroy(r.b); (void)hipEventDestroy(r.e); }
        open.clear();
        done.clear();
    }
};

int enqueue_train(ptmi_model *m, int T, hipStream_t s, TrainTracer *tr = nullptr) {
    TrainState *ts = m->train;
    const Resident *r = m->res;
    const Config &c = m->c;
    const int D = c.dim, H = c.hidden, L = c.n_layers, V = c.vocab, KV = c.kv_dim, NH = c.n_heads, hd = c.head_dim;
    const int QS = D + 2 * KV, R = T - 1, kv_mul = c.n_heads / c.n_kv_heads;
    const float scale = host_scale(hd);
    const long TD = (long)T * D;
    auto G = [&](const float *p) { return ts->gmem + (p - r->mem); };   // grad of a weight tensor
    int st;
    // span markers for the traced step (no-ops otherwise)
#define SPAN(name_, cat_, layer_) \
    do { if (tr && (st = tr->begin(name_, cat_, layer_))) return st; } while (0)
#define SPAN_END() \
    do { if (tr && (st = tr->end())) return st; } while (0)
    const size_t att_lds = (size_t)T * sizeof(float);
    // G lanes per head row: the smallest of 8/16/32 with 4*G >= head_dim
    const int hd4 = hd / 4;
    auto attn_fwd = hd4 <= 8 ? k_attn_fwd<8> : hd4 <= 16 ? k_attn_fwd<16> : k_attn_fwd<32>;
    auto attn_bwd_rows = hd4 <= 8 ? k_attn_bwd_rows<8> : hd4 <= 16 ? k_attn_bwd_rows<16> : k_attn_bwd_rows<32>;
    auto attn_bwd_cols = hd4 <= 8 ? k_attn_bwd_cols<8> : hd4 <= 16 ? k_attn_bwd_cols<16> : k_attn_bwd_cols<32>;
    // The matrix-core attention kernels when head_dim is a multiple of 16 (up
    // to 128), a row fits the softmax's registers and the LDS fits in 64 KB;
    // otherwise the per-position ones.
    using MfFwd = void (*)(const float *, float *, float *, int, int, int, float, int);
    using MfRows = void (*)(const float *, const float *, float *, const float *, const float *, float *, float *, int,
                            int, int, int, float,
                            int);
    using MfCols = void (*)(const float *, const float *, const float *, const float *, float *, int, int, int, int);
    static const MfFwd mf_fwd[8] = {k_attn_fwd_mfma<1>, k_attn_fwd_mfma<2>, k_attn_fwd_mfma<3>, k_attn_fwd_mfma<4>,
                                    k_attn_fwd_mfma<5>, k_attn_fwd_mfma<6>, k_attn_fwd_mfma<7>, k_attn_fwd_mfma<8>};
    static const MfRows mf_rows[8] = {k_attn_bwd_rows_mfma<1>, k_attn_bwd_rows_mfma<2>, k_attn_bwd_rows_mfma<3>,
                                      k_attn_bwd_rows_mfma<4>, k_attn_bwd_rows_mfma<5>, k_attn_bwd_rows_mfma<6>,
                                      k_attn_bwd_rows_mfma<7>, k_attn_bwd_rows_mfma<8>};
    static const MfCols mf_cols[8] = {k_attn_bwd_cols_mfma<1>, k_attn_bwd_cols_mfma<2>, k_attn_bwd_cols_mfma<3>,
                                      k_attn_bwd_cols_mfma<4>, k_attn_bwd_cols_mfma<5>, k_attn_bwd_cols_mfma<6>,
                                      k_attn_bwd_cols_mfma<7>, k_attn_bwd_cols_mfma<8>};
    const int HQ = hd / 16, pitch = (T + 15) / 16 * 16 + 4;
    const size_t mf_lds = std::max<size_t>((size_t)16 * pitch, (size_t)kMW * 16 * hd) * sizeof(float);
    const size_t mc_lds = (size_t)kMW * 16 * hd * sizeof(float);
    const bool mfma_attn =
        hd % 16 == 0 && HQ >= 1 && HQ <= 8 && KV == D && T <= 256 * kAttnChunks && mf_lds <= 65536;

    // pt_zero_grads (pt_train.c:425-427) is implicit: every gradient below is
    // written, not accumulated, by the one kernel that produces it (0 + v is
    // v), and gradient words no kernel produces stay at their initial zero.
    // The one accumulation is the embedding's: with the classifier tied to
    // it, the classifier's dW (written first) is its starting value;
    // untied, its rows are cleared here.
    // RMSNorm rows: one wave per row when D % 4 == 0 and D <= 2048, else one
    // block per row.
    using NormFn = void (*)(float *, const float *, float *, int, int, SplitK, const float *, const int *,
                            const float *, unsigned *);
    using NormBwdFn = void (*)(float *, const float *, float *, const float *, const float *, float *, int, int, SplitK);
    static const NormFn norm_w[8] = {k_rmsnorm_rows_w<1>, k_rmsnorm_rows_w<2>, k_rmsnorm_rows_w<3>,
                                     k_rmsnorm_rows_w<4>, k_rmsnorm_rows_w<5>, k_rmsnorm_rows_w<6>,
                                     k_rmsnorm_rows_w<7>, k_rmsnorm_rows_w<8>};
    static const NormBwdFn norm_bwd_w[8] = {k_rmsnorm_bwd_rows_w<1>, k_rmsnorm_bwd_rows_w<2>, k_rmsnorm_bwd_rows_w<3>,
                                            k_rmsnorm_bwd_rows_w<4>, k_rmsnorm_bwd_rows_w<5>, k_rmsnorm_bwd_rows_w<6>,
                                            k_rmsnorm_bwd_rows_w<7>, k_rmsnorm_bwd_rows_w<8>};
    const int nv = (D + 255) / 256;
    const bool wave_norm = D % 4 == 0 && nv <= 8;
    // embed: gather the rows from the embedding table first (layer 0)
    auto norm_fwd = [&](float *in, const float *w, float *out, SplitK pk, const float *cin, bool embed) {
        if (wave_norm) {
            hipLaunchKernelGGL(norm_w[nv - 1], dim3(T), dim3(64), 0, s, in, w, out, T, D, pk, cin,
                               embed ? ts->tok : nullptr, r->emb, ts->tok_bits);
        } else {
            if (embed) hipLaunchKernelGGL(k_embed_rows, dim3(T), dim3(256), 0, s, ts->tok, r->emb, in, D, ts->tok_bits,
                                          T - 1);
            hipLaunchKernelGGL(k_rmsnorm_rows, dim3(T), dim3(256), 0, s, in, w, out, D, pk, cin);
        }
    };
    // RMSNorm then an NT GEMM with a fused epilogue, C = epi(rmsnorm(x) . W^T):
    // the norm runs inside the GEMM's A loads when launch_gemm can fuse it
    // (the first N tile's blocks then store x and the normalized rows as
    // the norm kernel would), else as its own launch first.
    auto norm_gemm = [&](float *in, const float *w, float *out, SplitK pk, const float *cin, bool embed,
                         const float *W, int N, float *C, const GemmEpi *epi) -> int {
        GemmNorm nm = {};
        nm.kind = embed ? GEMM_NORM_EMBED : pk.splits > 0 ? GEMM_NORM_SPLITS : GEMM_NORM_PLAIN;
        nm.w = w; nm.pk = pk; nm.cin = cin;
        nm.tok = ts->tok; nm.emb = r->emb; nm.tok_bits = ts->tok_bits;
        nm.x_out = in; nm.xn_out = out;
        if (wave_norm && (ts->fuse_norm >> (nm.kind - 1) & 1) && gemm_norm_fusable(T, N, D, in, D, W, D, epi->kind, nm))
            return gemm(s, ts, 2, in, D, W, D, C, N, T, N, D, 0, nullptr, nullptr, epi, &nm);
        norm_fwd(in, w, out, pk, cin, embed);
        return gemm(s, ts, 2, out, D, W, D, C, N, T, N, D, 0, nullptr, nullptr, epi);
    };
    const bool tied = r->wcls == r->emb;
    SPAN("train_step", "train", -1);                      // pt.c:339-364
    SPAN("zero_grads", "train", -1);
    if (!tied) fill0(s, G(r->emb), (long)V * D);
    SPAN_END();
    // ── forward ──
    // Spans follow pt_train.c's (pt_forward_train :171-329): the embedding
    // gather runs inside layer 0's first RMSNorm, so "embedding" is empty.
    SPAN("forward", "fwd", -1);
    SPAN("embedding", "fwd", -1);
    SPAN_END();
    // A split-K w2 GEMM leaves its partial sums; the next RMSNorm completes
    // the residual stream row (adding the GEMM's residual input) and stores it.
    SplitK pend = {};
    const float *pend_cin = nullptr;
    const SplitK none = {};
    for (int l = 0; l < L; l++) {
        float *rin = ts->res + l * TD, *rmid = ts->res_att + l * TD, *rout = ts->res + (l + 1) * TD;
        float *xa = ts->xb_att + l * TD, *qkv = ts->qkv + (long)l * T * QS, *att = ts->att + (long)l * NH * T * T;
        float *ao = ts->att_out + l * TD, *xf = ts->xb_ffn + l * TD, *h13 = ts->h13 + (long)l * T * 2 * H;
        SPAN("layer", "fwd", l);
        SPAN("qkv", "fwd", l);
        // qkv = rmsnorm(x) . Wqkv^T with RoPE on the q and k columns in the GEMM's epilogue
        const GemmEpi rope = {GEMM_EPI_ROPE, nullptr, 0, D, hd};
        if ((st = norm_gemm(rin, r->rms_att + (long)l * D, xa, pend, pend_cin, l == 0, r->wqkv + (long)l * QS * D, QS,
                            qkv, &rope)))
            return st;
        SPAN_END();
        SPAN("attention", "fwd", l);
        if (mfma_attn)
            hipLaunchKernelGGL(mf_fwd[HQ - 1], dim3((T + kAttnRows - 1) / kAttnRows, NH), dim3(kMT), mf_lds, s, qkv, att,
                               ao, T, D, QS, scale, pitch);
        else
            hipLaunchKernelGGL(attn_fwd, dim3(T, NH), dim3(kAttnThreads), att_lds, s, qkv, att, ao, T, D, QS, KV, hd,
                               kv_mul, scale);
        // residual: rmid = rin + att_out . Wo^T (inside the attention span,
        // as pt_train.c:222-258 keeps the Wo matvecs)
        if ((st = gemm(s, ts, 2, ao, D, r->wo + (long)l * D * D, D, rmid, D, T, D, D, 1, rin))) return st;
        SPAN_END();
        SPAN("ffn", "fwd", l);
        // h13 = rmsnorm(x) . W13^T (rows interleaved w1/w3), sh = silu(h1)*h3 in the GEMM's epilogue
        const GemmEpi swiglu = {GEMM_EPI_SWIGLU, ts->sh, H, 0, 0};
        if ((st = norm_gemm(rmid, r->rms_ffn + (long)l * D, xf, none, nullptr, false, r->w13 + (long)l * 2 * H * D,
                            2 * H, h13, &swiglu)))
            return st;
        if ((st = gemm(s, ts, 2, ts->sh, H, r->w2 + (long)l * D * H, H, rout, D, T, D, H, 1, rmid, &pend))) return st;
        pend_cin = rmid;
        SPAN_END();
        SPAN_END();
    }
    SPAN("classifier", "fwd", -1);
    norm_fwd(ts->res + L * TD, r->rms_final, ts->x_final, pend, pend_cin, false);
    if ((st = gemm(s, ts, 2, ts->x_final, D, r->wcls, D, ts->logits, V, T, V, D, 0))) return st;
    SPAN_END();
    SPAN("loss", "fwd", -1);
    {
        using LossFn = void (*)(float *, const int *, int, int, float, float *);
        const int slots = (V / 4 + kLossThreads - 1) / kLossThreads;
        const LossFn loss = V % 4 ? k_loss_rows
                            : slots <= 1 ? k_loss_rows_reg<1>
                            : slots <= 2 ? k_loss_rows_reg<2>
                            : slots <= 4 ? k_loss_rows_reg<4>
                            : slots <= 8 ? k_loss_rows_reg<8>
                                         : k_loss_rows;
        hipLaunchKernelGGL(loss, dim3(T), dim3(kLossThreads), 0, s, ts->logits, ts->tok, T, V, 1.0f / (float)(T - 1),
                           ts->row_loss);
    }
    PTMI_HIP(hipGetLastError());

    SPAN_END();
    SPAN_END();
    // ── backward ── (ts->logits now holds d_logits)
    // The dX chain runs here; the weight gradients (25 TN GEMMs and 2L+1
    // RMSNorm dW reductions) only read buffers written once per step, so
    // they run afterwards as two grouped launches (descriptor tables built
    // by train_descriptors for this T).
    auto dres = [&](int k) { return ts->d_res + (long)k * TD; };
    auto dxb = [&](int k) { return ts->d_xb + (long)k * TD; };
    int v = 0;                                            // d_res version
    SplitK pk = {};                                       // split-K partials of d_xb[v], if deferred
    auto norm_bwd = [&](const float *x, const float *w) {
        // d_res[v+1] = d_res[v] + rmsnorm_backward(d_xb[v]); inverse norms kept per norm
        if (wave_norm)
            hipLaunchKernelGGL(norm_bwd_w[nv - 1], dim3(R), dim3(64), 0, s, dres(v + 1),
                               v ? dres(v) : nullptr, dxb(v), x, w, ts->row_inv + (long)v * T, R, D, pk);
        else
            hipLaunchKernelGGL(k_rmsnorm_bwd_rows, dim3(R), dim3(256), 0, s, dres(v + 1), v ? dres(v) : nullptr,
                               dxb(v), x, w, ts->row_inv + (long)v * T, D, pk);
        pk = SplitK{};
        v++;
    };
    SPAN("backward", "bwd", -1);                          // pt_backward, pt_train.c:549-866
    SPAN("classifier", "bwd", -1);                        // pt_train.c:585-653
    // The reference transposes Wcls on the host here (:590-594); the NN
    // GEMM reads Wcls as stored, so the span is empty.
    SPAN("cls_transpose", "bwd", -1);
    SPAN_END();
    if ((st = gemm(s, ts, 0, ts->logits, V, r->wcls, D, dxb(0), D, R, D, V, 0, nullptr, &pk))) return st;
    norm_bwd(ts->res + L * TD, r->rms_final);
    // Traced, the classifier's weight gradient (entry 0 of the grouped
    // table, with its fused SGD step) runs here as its own launch, under
    // cls_weight_grad (:644-652).  No later kernel of the step reads Wcls,
    // and the tied embedding rows are still left to the embedding backward,
    // so every value is the same as in the grouped launch.
    if (tr) {
        SPAN("cls_weight_grad", "bwd", -1);
        if ((st = launch_gemm_tn_group(ts->dw_desc, 0, 1, ts->dw_cls_tiles, ts->dw_vec, s))) return st;
        SPAN_END();
    }
    SPAN_END();
    for (int l = L - 1; l >= 0; l--) {
        const float *rin = ts->res + l * TD, *rmid = ts->res_att + l * TD;
        const float *qkv = ts->qkv + (long)l * T * QS, *att = ts->att + (long)l * NH * T * T;
        const float *h13 = ts->h13 + (long)l * T * 2 * H;
        const float *w2 = r->w2 + (long)l * D * H, *w13 = r->w13 + (long)l * 2 * H * D;
        const float *wo = r->wo + (long)l * D * D, *wqkv = r->wqkv + (long)l * QS * D;
        float *dh13 = ts->d_h13 + (long)l * T * 2 * H, *shb = ts->shb + (long)l * T * H;
        float *dqkv = ts->d_qkv + (long)l * T * QS;
        // FFN
        // d_sh = d_res . W2, consumed in the GEMM's epilogue by the swiglu
        // backward: d_h13 (interleaved d_h1, d_h3) and shb = silu(h1)*h3
        SPAN("layer", "bwd", l);
        // the reference's per-layer host transposes (:669-680): none here
        SPAN("transpose", "bwd", l);
        SPAN_END();
        SPAN("ffn", "bwd", l);
        GemmEpi sgb = {GEMM_EPI_SWIGLU_BWD, dh13, 2 * H, 0, 0, shb, H, h13, 2 * H};
        if ((st = gemm(s, ts, 0, dres(v), D, w2, H, ts->d_sh, H, R, H, D, 0, nullptr, nullptr, &sgb))) return st;
        if ((st = gemm(s, ts, 0, dh13, 2 * H, w13, D, dxb(v), D, R, D, 2 * H, 0, nullptr, &pk))) return st;
        norm_bwd(rmid, r->rms_ffn + (long)l * D);
        SPAN_END();
        // Wo: d_aout = d_res . Wo, inside the matrix-core attention rows
        // kernel when D splits over its waves in whole MFMA k steps
        const bool wo_fused = mfma_attn && D % (4 * kMW) == 0;
        SPAN("wo", "bwd", l);
        if (!wo_fused && (st = gemm(s, ts, 0, dres(v), D, wo, D, ts->d_aout, D, R, D, D, 0))) return st;
        SPAN_END();
        // attention
        SPAN("attention", "bwd", l);
        if (mfma_attn) {
            hipLaunchKernelGGL(mf_rows[HQ - 1], dim3((R + kAttnRows - 1) / kAttnRows, NH), dim3(kMT), mf_lds, s, qkv,
                               att, ts->d_aout, wo_fused ? dres(v) : nullptr, wo, ts->ds, dqkv, T, R, D, QS, scale, pitch);
            hipLaunchKernelGGL(mf_cols[HQ - 1], dim3((R + 15) / 16, NH), dim3(kMT), mc_lds, s, qkv, att, ts->ds,
                               ts->d_aout, dqkv, T, R, D, QS);
        } else {
            hipLaunchKernelGGL(attn_bwd_rows, dim3(R, NH), dim3(kAttnThreads), att_lds, s, qkv, att, ts->d_aout, ts->ds,
                               ts->d_q, T, D, QS, KV, hd, kv_mul, scale);
            hipLaunchKernelGGL(attn_bwd_cols, dim3(R, NH), dim3(kAttnThreads), 2 * att_lds, s, qkv, att, ts->ds,
                               ts->d_aout, ts->d_k, ts->d_v, T, R, D, QS, KV, hd, kv_mul);
            hipLaunchKernelGGL(k_rope_bwd_pack, dim3(blocks_for((long)R * D / 2, 256)), dim3(256), 0, s, ts->d_q,
                               ts->d_k, ts->d_v, dqkv, R, D, KV, QS, hd);
        }
        PTMI_HIP(hipGetLastError());
        SPAN_END();
        // QKV
        SPAN("qkv", "bwd", l);
        if ((st = gemm(s, ts, 0, dqkv, QS, wqkv, D, dxb(v), D, R, D, QS, 0, nullptr, &pk))) return st;
        norm_bwd(rin, r->rms_att + (long)l * D);
        SPAN_END();
        SPAN_END();
    }
    PTMI_HIP(hipGetLastError());
    // weight gradients: every TN GEMM in one launch (traced: the layers'
    // ones, under a span the reference does not have, since it computes
    // each layer's dW inside that layer's spans), every RMSNorm dW in one
    if (tr) {
        SPAN("weight_grads", "bwd", -1);
        if ((st = launch_gemm_tn_group(ts->dw_desc, 1, ts->n_dw, ts->dw_tiles - ts->dw_cls_tiles, ts->dw_vec, s)))
            return st;
        SPAN_END();
    } else if ((st = launch_gemm_tn_group(ts->dw_desc, 0, ts->n_dw, ts->dw_tiles, ts->dw_vec, s))) {
        return st;
    }
    SPAN("embedding", "bwd", -1);
    // every RMSNorm dW, the embedding backward and the mean loss in one
    {
        const int cb = (D + 63) / 64, nn = (2 * L + 1) * cb;
        hipLaunchKernelGGL(k_step_tail, dim3((unsigned)(nn + R + 1)), dim3(1024), (size_t)(R + 31) / 32 * sizeof(unsigned),
                           s, reinterpret_cast<const NormDw *>(ts->nd_desc), cb, nn, R, D, ts->tok, dres(v), G(r->emb),
                           r->emb, ts->tok_bits, ts->lr, ts->row_loss, ts->loss);
        PTMI_HIP(hipGetLastError());
    }
    SPAN_END();
    SPAN_END();                                           // backward
    // SGD (pt_sgd_update, pt_train.c:870-896): every update happened in the
    // kernel that wrote its gradient, so its span is empty.
    SPAN("sgd", "train", -1);
    SPAN_END();
    SPAN_END();                                           // train_step
    return PTMI_OK;
#undef SPAN
#undef SPAN_END
}

}  // namespace

}  // namespace ptmi

using namespace ptmi;

extern "C" {

// Checks a train step's arguments, uploads its tokens and learning rate and
// builds the descriptor tables for T.
static int train_prepare(ptmi_model_t *m, const int *tokens, int T, float lr) {
    if (!m || !tokens) return set_error(PTMI_ERR_ARG, "NULL argument");
    if (!m->train) return set_error(PTMI_ERR_STATE, "model created with max_T = 0 (no training buffers)");
    if (T < 2 || T > m->train->T_max) return set_error(PTMI_ERR_ARG, "T=%d outside [2, max_T=%d]", T, m->train->T_max);
    for (int i = 0; i < T; i++)
        if (tokens[i] < 0 || tokens[i] >= m->c.vocab) return set_error(PTMI_ERR_ARG, "tokens[%d]=%d out of range", i, tokens[i]);
    hipStream_t s = lib_stream();
    TrainState *ts = m->train;
    // a step that returned early may have left its copy in flight
    if (ts->pin_busy) PTMI_HIP(hipStreamSynchronize(s));
    memcpy(ts->pin, tokens, (size_t)T * sizeof(int));
    ts->pin[ts->lr_off] = lr;
    ts->pin_busy = true;
    PTMI_HIP(hipMemcpyAsync(ts->tok, ts->pin, (size_t)(ts->lr_off + 1) * sizeof(float), hipMemcpyHostToDevice, s));
    return train_descriptors(m, T);
}

int ptmi_model_train_step(ptmi_model_t *m, const int *tokens, int T, float lr, float *loss) {
    int st = train_prepare(m, tokens, T, lr);
    if (st) return st;
    hipStream_t s = lib_stream();
    TrainState *ts = m->train;
    if (ts->eager) {
        if ((st = enqueue_train(m, T, s))) return st;
    } else {
        if (ts->graph_T != T) {                    // capture the step for this T
            if (ts->exec) (void)hipGraphExecDestroy(ts->exec);
            if (ts->graph) (void)hipGraphDestroy(ts->graph);
            ts->exec = nullptr;
            ts->graph = nullptr;
            ts->graph_T = 0;
            PTMI_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            st = enqueue_train(m, T, s);
            hipGraph_t graph = nullptr;
            const hipError_t e = hipStreamEndCapture(s, &graph);
            if (st) { if (graph) (void)hipGraphDestroy(graph); return st; }
            if (e != hipSuccess) return hip_check(e, "hipStreamEndCapture(train step)");
            hipGraphExec_t exec = nullptr;
            const hipError_t e2 = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            if (e2 != hipSuccess) { (void)hipGraphDestroy(graph); return hip_check(e2, "hipGraphInstantiate(train step)"); }
            ts->graph = graph;
            ts->exec = exec;
            ts->graph_T = T;
        }
        PTMI_HIP(hipGraphLaunch(ts->exec, s));
    }
    float *l = ts->pin + ts->lr_off + 1;
    PTMI_HIP(hipMemcpyAsync(l, ts->loss, sizeof(float), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    ts->pin_busy = false;
    if (loss) *loss = *l;
    return PTMI_OK;
}

static float *ts_sink(ptmi_model_t *m) { return m->train->ws; }

int ptmi_model_train_step_trace(ptmi_model_t *m, const int *tokens, int T, float lr, float *loss,
                                ptmi_span_t *spans, int max_spans, int *n_spans) {
    if (!n_spans || (max_spans > 0 && !spans) || max_spans < 0) return set_error(PTMI_ERR_ARG, "bad span buffer");
    *n_spans = 0;
    int st = train_prepare(m, tokens, T, lr);
    if (st) return st;
    hipStream_t s = lib_stream();
    TrainTracer tr;
    tr.s = s;
    // The traced step is enqueued eagerly (events do not time graph nodes)
    // behind a bounded busy kernel that holds the stream while the host
    // enqueues it, so its kernels then run back to back and the spans time
    // device work, not the host's enqueue gaps.
    hipLaunchKernelGGL(k_hold, dim3(1), dim3(64), 0, s, ts_sink(m), kHoldIters);
    PTMI_HIP(hipGetLastError());
    st = enqueue_train(m, T, s, &tr);
    float l = 0.0f;
    if (!st) {
        const hipError_t e = hipMemcpyAsync(&l, m->train->loss, sizeof(float), hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) st = hip_check(e, "loss copy");
    }
    const hipError_t es = hipStreamSynchronize(s);
    if (es == hipSuccess) m->train->pin_busy = false;
    if (!st && es != hipSuccess) st = hip_check(es, "hipStreamSynchronize(traced train step)");
    if (!st && !tr.open.empty()) st = set_error(PTMI_ERR_STATE, "unclosed trace span %s", tr.open.back().name);
    const TrainTracer::Rec *root = nullptr;
    for (const auto &r : tr.done)
        if (r.depth == 0) root = &r;
    if (!st && !root) st = set_error(PTMI_ERR_STATE, "traced step has no root span");
    if (!st) {
        *n_spans = (int)tr.done.size();
        if (max_spans < *n_spans) {
            st = set_error(PTMI_ERR_ARG, "span buffer holds %d, the step has %d spans", max_spans, *n_spans);
        } else {
            for (size_t i = 0; i < tr.done.size() && !st; i++) {
                const auto &r = tr.done[i];
                float a = 0.0f, d = 0.0f;
                hipError_t e = hipEventElapsedTime(&a, root->b, r.b);
                if (e == hipSuccess) e = hipEventElapsedTime(&d, r.b, r.e);
                if (e != hipSuccess) { st = hip_check(e, "hipEventElapsedTime(trace span)"); break; }
                spans[i] = ptmi_span_t{r.name, r.cat, r.layer, r.depth, 1e3 * a, 1e3 * d};
            }
        }
    }
    tr.release();
    if (!st && loss) *loss = l;
    return st;
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
