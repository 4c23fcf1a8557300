// Device-resident decode step (pt_forward_step, pitorch/pt.c:267-271 over
// pt_forward, pitorch/model/llama2.c:127-206) captured once as a hipGraph.
//
// Per layer, five launches:
//   1. QKV matvec   : RMSNorm prologue (+ embedding gather on layer 0),
//                     RoPE epilogue, K/V written straight into the cache
//   2. attention    : (head, chunk of positions) workgroups, each leaving
//                     its chunk's partial softmax sums
//   3. Wo matvec    : attention-combine prologue (merges the chunks of every
//                     head), residual-add epilogue
//   4. w1|w3 matvec : RMSNorm prologue, rows interleaved, SwiGLU epilogue
//   5. w2 matvec    : residual-add epilogue
// then the classifier matvec (final RMSNorm prologue) and one argmax
// workgroup that also advances the position and picks the next input token.
#include "ptmi_model.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <vector>
#include <type_traits>

namespace ptmi {

// att_scale = 1/pt_sqrtf(head_dim) (llama2.c:137), evaluated on the host
// with the reference's seed + 3 Newton steps (pt_math.c:92-102).
float host_att_scale(int head_dim) {
    const float x = (float)head_dim;
    uint32_t u;
    memcpy(&u, &x, 4);
    u = 0x1fbd1df5u + (u >> 1);
    float y;
    memcpy(&y, &u, 4);
    for (int i = 0; i < 3; i++) y = 0.5f * (y + x / y);
    return 1.0f / y;
}

namespace {

struct AttnParams {
    const float *q;         // [D] post-RoPE query
    const float *kc, *vc;   // this layer's caches [seq_len, kv_dim]
    float *part_o;          // [heads][chunks][head_dim] unnormalised weighted V sums
    float *part_ml;         // [heads][chunks][2] chunk max, chunk sum of e^(s - max)
    const DecodeCtl *ctl;
    int head_dim, kv_dim, kv_mul, n_heads, chunk, n_chunks;
    float scale;
    PrefetchDesc pf;        // blocks past n_heads*n_chunks prefetch the next weights
};

__device__ __forceinline__ float dot4(float4 a, float4 b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    return fmaf(a.w, b.w, acc);
}

// 8 waves of 4 loads in flight cover a 128-position chunk in one batch
// (G = 16): 3664 tok/s against 3589 for 4 waves of 8 and 3376 for 16 of 2.
constexpr int kAttnWaves = 8;
constexpr int kAttnUnroll = 4;
constexpr int kMaxAttnChunk = 512;

// llama2.c:153-177, split over (head, chunk of positions) workgroups so the
// KV-cache read is spread over many CUs (one CU streams only ~30 GB/s).
// Each workgroup leaves its chunk's max m, sum l = sum e^(s-m) and the
// unnormalised sum o = sum e^(s-m) v; the Wo matvec combines the chunks.
// G lanes hold one K/V row (G*4 >= head_dim); a wave's load covers 64/G
// positions and kAttnUnroll loads are in flight before any is consumed.
template <int G>
__global__ __launch_bounds__(kAttnWaves * 64) void k_attn_chunk(AttnParams a) {
    constexpr int RPI = 64 / G;
    constexpr int BATCH = RPI * kAttnUnroll;
    __shared__ float sc[kMaxAttnChunk];
    __shared__ float red[kAttnWaves][kMaxHeadDim];
    __shared__ float wred[kAttnWaves];

    // The position (a scalar load) goes out first; the compute path's
    // arguments are fetched in the same batch as the prefetch test.
    const int n = a.ctl->pos + 1;
    kernarg_batch(a.q, a.kc, a.vc, a.part_o, a.part_ml, a.head_dim, a.kv_dim, a.kv_mul, a.chunk, a.scale);
    if ((int)blockIdx.x >= a.n_heads * a.n_chunks) {
        run_prefetch(a.pf);
        return;
    }
    const int h = blockIdx.x % a.n_heads, c = blockIdx.x / a.n_heads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int slot = lane / G, sub = lane % G;
    const int hd = a.head_dim, hd4 = hd >> 2;
    const bool has = sub < hd4;
    const int sub_c = has ? sub : 0;
    // q does not depend on the position: its load overlaps the pos fetch.
    float4 q4 = reinterpret_cast<const float4 *>(a.q + h * hd)[sub_c];
    const int t0 = c * a.chunk;
    if (t0 >= n) return;                               // uniform per block
    const int t1 = min(t0 + a.chunk, n);
    const long ko = (long)(h / a.kv_mul) * hd;
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!has) q4 = zero4;
    const int cnt = t1 - t0;
    const float4 *kbase = reinterpret_cast<const float4 *>(a.kc + ko) + sub_c;
    const float4 *vbase = reinterpret_cast<const float4 *>(a.vc + ko) + sub_c;
    const long row4 = a.kv_dim >> 2;                     // float4 per cache row

    // K/V rows with nontemporal loads: read once per step, they should not
    // evict the w1|w3 weights this launch's prefetch blocks stage in L2.
    typedef float fx4 __attribute__((ext_vector_type(4)));
    auto load_rows = [&](const float4 *src, int base, float4 (&dst)[kAttnUnroll]) {
#pragma unroll
        for (int u = 0; u < kAttnUnroll; u++) {
            const fx4 t = __builtin_nontemporal_load(
                reinterpret_cast<const fx4 *>(src + (long)min(base + u * RPI + slot, t1 - 1) * row4));
            dst[u] = make_float4(t.x, t.y, t.z, t.w);
        }
    };
    auto score_rows = [&](int base, const float4 (&k4)[kAttnUnroll]) {
#pragma unroll
        for (int u = 0; u < kAttnUnroll; u++) {
            float s = has ? dot4(k4[u], q4, 0.0f) : 0.0f;
            s = group_sum<G>(s);
            const int t = base + u * RPI + slot;
            if (sub == 0 && t < t1) sc[t - t0] = s * a.scale;
        }
    };
    // chunk softmax over sc[0..cnt): sc <- e^(s - max); returns the max,
    // leaves each wave's partial sum in wred
    auto softmax = [&]() {
        __syncthreads();
        float mx = -INFINITY;
        for (int i = tid; i < cnt; i += kAttnWaves * 64) mx = fmaxf(mx, sc[i]);
        mx = group_max<64>(mx);
        if (lane == 0) wred[wave] = mx;
        __syncthreads();
        mx = wred[0];
#pragma unroll
        for (int w = 1; w < kAttnWaves; w++) mx = fmaxf(mx, wred[w]);
        __syncthreads();
        float sum = 0.0f;
        for (int i = tid; i < cnt; i += kAttnWaves * 64) {
            const float e = d_expf(sc[i] - mx);
            sc[i] = e;
            sum += e;
        }
        sum = group_sum<64>(sum);
        if (lane == 0) wred[wave] = sum;
        __syncthreads();
        return mx;
    };
    auto accumulate = [&](int base, const float4 (&v4)[kAttnUnroll], float4 &acc) {
#pragma unroll
        for (int u = 0; u < kAttnUnroll; u++) {
            const int t = base + u * RPI + slot;
            const float e = t < t1 ? sc[t - t0] : 0.0f;
            acc.x = fmaf(e, v4[u].x, acc.x);
            acc.y = fmaf(e, v4[u].y, acc.y);
            acc.z = fmaf(e, v4[u].z, acc.z);
            acc.w = fmaf(e, v4[u].w, acc.w);
        }
    };

    float4 acc = zero4;
    float mx;
    if (cnt <= kAttnWaves * BATCH) {
        // One batch per wave: the V rows are loaded together with the K
        // rows, so the softmax does not wait for a second round trip.
        // Waves past the chunk's end re-read row t1-1 and add nothing.
        const int base = t0 + wave * BATCH;
        float4 k4[kAttnUnroll], v4[kAttnUnroll];
        load_rows(kbase, base, k4);
        load_rows(vbase, base, v4);
        score_rows(base, k4);
        mx = softmax();
        accumulate(base, v4, acc);
    } else {
        for (int base = t0 + wave * BATCH; base < t1; base += kAttnWaves * BATCH) {
            float4 k4[kAttnUnroll];
            load_rows(kbase, base, k4);
            score_rows(base, k4);
        }
        mx = softmax();
        for (int base = t0 + wave * BATCH; base < t1; base += kAttnWaves * BATCH) {
            float4 v4[kAttnUnroll];
            load_rows(vbase, base, v4);
            accumulate(base, v4, acc);
        }
    }
    // sum over the wave's slots (lanes with equal lane % G): rows of 16
    // pair i with i+8 by a DPP rotate (G = 8), then the permlane swaps
    static_assert(G == 8 || G == 16 || G == 32, "lanes per row");
    auto slot_sum = [](float v) {
        if constexpr (G == 8)
            v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
        if constexpr (G <= 16) v = xsum16(v);
        return xsum32(v);
    };
    acc.x = slot_sum(acc.x);
    acc.y = slot_sum(acc.y);
    acc.z = slot_sum(acc.z);
    acc.w = slot_sum(acc.w);
    if (slot == 0 && has) {
        red[wave][4 * sub + 0] = acc.x;
        red[wave][4 * sub + 1] = acc.y;
        red[wave][4 * sub + 2] = acc.z;
        red[wave][4 * sub + 3] = acc.w;
    }
    __syncthreads();
    const long slot_id = (long)h * a.n_chunks + c;
    if (tid < hd) {
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; w++) o += red[w][tid];
        a.part_o[slot_id * hd + tid] = o;
    }
    if (tid == 0) {
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; w++) l += wred[w];
        a.part_ml[2 * slot_id] = mx;
        a.part_ml[2 * slot_id + 1] = l;
    }
}

// argmax (pt_ops.c:65-70: the first index of the maximum; a NaN at index 0
// makes it 0, other NaNs never win) + step bookkeeping (pt.c:269 pos++,
// pt_text.c:344-350 prefill forcing).  float4 loads, eight in flight per
// thread; each thread scans ascending indices, ties resolve to the smaller
// index.
__global__ __launch_bounds__(1024) void k_argmax_step(const float *logits, int n, DecodeCtl *ctl,
                                                      const int *prompt, int *out_tokens, PrefetchDesc pf) {
    if (blockIdx.x > 0) {
        run_prefetch(pf);
        return;
    }
    __shared__ float sv[16];
    __shared__ int si[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    const int n4 = n >> 2;
    const float4 *l4 = reinterpret_cast<const float4 *>(logits);
    for (int base = tid; base < n4; base += 8 * 1024) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = l4[min(base + u * 1024, n4 - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i4 = base + u * 1024;
            if (i4 < n4) {
                if (v[u].x > bv) { bv = v[u].x; bi = 4 * i4; }
                if (v[u].y > bv) { bv = v[u].y; bi = 4 * i4 + 1; }
                if (v[u].z > bv) { bv = v[u].z; bi = 4 * i4 + 2; }
                if (v[u].w > bv) { bv = v[u].w; bi = 4 * i4 + 3; }
            }
        }
    }
    for (int i = 4 * n4 + tid; i < n; i += 1024) {
        const float v = logits[i];
        if (v > bv) { bv = v; bi = i; }
    }
    wave_argmax(bv, bi);
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++) take_max(bv, bi, sv[w], si[w]);
        if (bi == 0x7fffffff || logits[0] != logits[0]) bi = 0;   // nothing above -inf, or a NaN first: 0
        const int pos = ctl->pos;
        const int next = (pos < ctl->n_prompt - 1) ? prompt[pos + 1] : bi;
        ctl->next = bi;
        ctl->tok_in = next;
        ctl->pos = pos + 1;
        if (out_tokens) out_tokens[pos] = next;
    }
}

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Optional per-launch HIP events (eager profiling runs only): each launch
// gets a start/stop pair timestamped by the command processor around the
// kernel itself (hipExtLaunchKernelGGL), i.e. the kernel's own duration.
struct StepTimer {
    std::vector<hipEvent_t> ev;     // 2 per launch
    std::vector<int> role;
    size_t used = 0;
    int next(int r, hipEvent_t *e0, hipEvent_t *e1) {
        if (used + 2 > ev.size()) {
            hipEvent_t a, b;
            PTMI_HIP(hipEventCreate(&a));
            PTMI_HIP(hipEventCreate(&b));
            ev.push_back(a);
            ev.push_back(b);
            role.push_back(0);
        }
        role[used / 2] = r;
        *e0 = ev[used];
        *e1 = ev[used + 1];
        used += 2;
        return PTMI_OK;
    }
    ~StepTimer() {
        for (hipEvent_t e : ev) (void)hipEventDestroy(e);
    }
};

#define TIMED(role_, launch_)                                   \
    do {                                                        \
        hipEvent_t e0 = nullptr, e1 = nullptr;                  \
        if (tm && (st = tm->next(role_, &e0, &e1))) return st;  \
        launch_;                                                \
    } while (0)

// Producer-side prefetch of consumer matvec weights W[rows, n] (ld = n).
// The producer's own grid is `first_block` blocks of `threads` threads.
PrefetchDesc pf_matvec(const ptmi_model *m, const float *W, int rows, int n, int pro, int epi, int first_block,
                       int threads) {
    if (!m->prefetch) return PrefetchDesc{};
    return prefetch_for(W, n, rows, n, pro, epi, first_block, threads, m->sink);
}

// The prefetch of producer `stage` (0 QKV, 1 attention, 2 Wo, 3 w1|w3,
// 4 w2, 5 classifier, 6 argmax) in layer l, per m->prefetch_plan; the
// producer's own grid is `first_block` blocks of `threads` threads.
PrefetchDesc pf_plan(const ptmi_model *m, int stage, int l, int first_block, int threads) {
    const Config &c = m->c;
    const Resident *r = m->res;
    const int D = c.dim, H = c.hidden, QR = c.dim + 2 * c.kv_dim, L = c.n_layers;
    const int ll = l < L ? l + 1 : 0;                 // the next layer (next token's first after the last)
    switch (m->prefetch_plan[stage]) {
    case 'o': return l < L ? pf_matvec(m, r->wo + (long)l * D * D, D, D, PRO_ATTN_COMBINE, EPI_RESIDUAL, first_block, threads) : PrefetchDesc{};
    case 'f': return l < L ? pf_matvec(m, r->w13 + (long)l * 2 * H * D, 2 * H, D, PRO_RMSNORM, EPI_SWIGLU, first_block, threads) : PrefetchDesc{};
    case 'd': return l < L ? pf_matvec(m, r->w2 + (long)l * D * H, D, H, PRO_NONE, EPI_RESIDUAL, first_block, threads) : PrefetchDesc{};
    case 'q': return pf_matvec(m, r->wqkv + (long)(ll < L ? ll : 0) * QR * D, QR, D, ll == 0 ? PRO_EMBED_RMSNORM : PRO_RMSNORM,
                               EPI_QKV_ROPE, first_block, threads);
    case 'O': return ll < L && ll > 0 ? pf_matvec(m, r->wo + (long)ll * D * D, D, D, PRO_ATTN_COMBINE, EPI_RESIDUAL, first_block, threads) : PrefetchDesc{};
    case 'F': return ll < L && ll > 0 ? pf_matvec(m, r->w13 + (long)ll * 2 * H * D, 2 * H, D, PRO_RMSNORM, EPI_SWIGLU, first_block, threads) : PrefetchDesc{};
    default: return PrefetchDesc{};
    }
}

// Enqueue one decode step on s (used both for capture and eager runs).
// A launch can carry extra blocks that read the weights of a later matvec
// (m->prefetch_plan): each kernel starts with an L2 invalidate, so the
// consumer then finds them in the memory-side MALL.
int enqueue_step(ptmi_model *m, hipStream_t s, StepTimer *tm = nullptr) {
    const Config &c = m->c;
    const Resident *r = m->res;
    const long D = c.dim, H = c.hidden, KV = c.kv_dim, S = c.seq_len;
    const int QR = (int)(D + 2 * KV);
    int st = PTMI_OK;
    if (m->step_mem) {                                    // the one-kernel step (or its windows)
        for (int w = 0; w < decode_step_windows(m) && st == PTMI_OK; w++) TIMED(7, st = launch_decode_step(m, w, s, e0, e1));
        return st;
    }
    for (int l = 0; l < c.n_layers; l++) {
        float *kc = m->kc + (long)l * S * KV, *vc = m->vc + (long)l * S * KV;
        MatvecParams p = {};
        p.W = r->wqkv + (long)l * (D + 2 * KV) * D; p.ld = D; p.rows = (int)(D + 2 * KV); p.n = (int)D;
        p.pro = l == 0 ? PRO_EMBED_RMSNORM : PRO_RMSNORM;
        p.x = l == 0 ? r->emb : m->x;
        p.token = &m->ctl->tok_in; p.x_out = m->x;
        p.norm_w = r->rms_att + l * D;
        p.y = m->q; p.epi = EPI_QKV_ROPE; p.pos = &m->ctl->pos;
        p.q_rows = (int)D; p.kv_rows = (int)KV; p.head_dim = c.head_dim; p.k_cache = kc; p.v_cache = vc;
        p.pf = pf_plan(m, 0, l, matvec_compute_blocks(QR, (int)D, p.pro, EPI_QKV_ROPE),
                       matvec_block_threads(QR, (int)D, p.pro, EPI_QKV_ROPE));
        TIMED(0, if ((st = launch_matvec(p, s, e0, e1))) return st);

        AttnParams a = {};
        a.q = m->q; a.kc = kc; a.vc = vc; a.part_o = m->part_o; a.part_ml = m->part_ml; a.ctl = m->ctl;
        a.head_dim = c.head_dim; a.kv_dim = (int)KV; a.kv_mul = c.n_heads / c.n_kv_heads;
        a.n_heads = c.n_heads; a.chunk = m->attn_chunk; a.n_chunks = m->attn_chunks;
        a.scale = host_att_scale(c.head_dim);
        const int hd4 = c.head_dim / 4;
        auto attn = hd4 <= 8 ? k_attn_chunk<8> : hd4 <= 16 ? k_attn_chunk<16> : k_attn_chunk<32>;
        const int attn_blocks = c.n_heads * m->attn_chunks;
        a.pf = pf_plan(m, 1, l, attn_blocks, kAttnWaves * 64);
        a.pf.first_block = attn_blocks;
        TIMED(1, launch_k(attn, dim3(attn_blocks + a.pf.blocks), dim3(kAttnWaves * 64), 0, s, e0, e1, a));
        PTMI_HIP(hipGetLastError());

        p = MatvecParams{};
        p.W = r->wo + (long)l * D * D; p.ld = D; p.rows = (int)D; p.n = (int)D;
        p.x = m->xb; p.y = m->x; p.pro = PRO_ATTN_COMBINE; p.epi = EPI_RESIDUAL;
        p.pos = &m->ctl->pos; p.att_o = m->part_o; p.att_ml = m->part_ml;
        p.att_chunks = m->attn_chunks; p.att_chunk = m->attn_chunk; p.att_heads = c.n_heads;
        p.pf = pf_plan(m, 2, l, matvec_compute_blocks((int)D, (int)D, PRO_ATTN_COMBINE, EPI_RESIDUAL),
                       matvec_block_threads((int)D, (int)D, PRO_ATTN_COMBINE, EPI_RESIDUAL));
        TIMED(2, if ((st = launch_matvec(p, s, e0, e1))) return st);

        p = MatvecParams{};
        p.W = r->w13 + (long)l * 2 * H * D; p.ld = D; p.rows = (int)(2 * H); p.n = (int)D;
        p.x = m->x; p.pro = PRO_RMSNORM; p.norm_w = r->rms_ffn + l * D;
        p.y = m->hb; p.epi = EPI_SWIGLU;
        p.pf = pf_plan(m, 3, l, matvec_compute_blocks((int)(2 * H), (int)D, PRO_RMSNORM, EPI_SWIGLU),
                       matvec_block_threads((int)(2 * H), (int)D, PRO_RMSNORM, EPI_SWIGLU));
        TIMED(3, if ((st = launch_matvec(p, s, e0, e1))) return st);

        p = MatvecParams{};
        p.W = r->w2 + (long)l * D * H; p.ld = H; p.rows = (int)D; p.n = (int)H;
        p.x = m->hb; p.y = m->x; p.pro = PRO_NONE; p.epi = EPI_RESIDUAL;
        p.pf = pf_plan(m, 4, l, matvec_compute_blocks((int)D, (int)H, PRO_NONE, EPI_RESIDUAL),
                       matvec_block_threads((int)D, (int)H, PRO_NONE, EPI_RESIDUAL));
        TIMED(4, if ((st = launch_matvec(p, s, e0, e1))) return st);
    }
    MatvecParams p = {};
    p.W = r->wcls; p.ld = D; p.rows = c.vocab; p.n = (int)D;
    p.x = m->x; p.pro = PRO_RMSNORM; p.norm_w = r->rms_final; p.y = m->logits; p.epi = EPI_STORE;
    p.pf = pf_plan(m, 5, c.n_layers, matvec_compute_blocks(c.vocab, (int)D, PRO_RMSNORM, EPI_STORE),
                   matvec_block_threads(c.vocab, (int)D, PRO_RMSNORM, EPI_STORE));
    TIMED(5, if ((st = launch_matvec(p, s, e0, e1))) return st);
    PrefetchDesc apf = pf_plan(m, 6, c.n_layers, 1, 1024);
    apf.first_block = 1;
    TIMED(6, launch_k(k_argmax_step, dim3(1 + apf.blocks), dim3(1024), 0, s, e0, e1, m->logits, c.vocab, m->ctl,
                      m->prompt, m->out_tokens, apf));
    PTMI_HIP(hipGetLastError());
    return PTMI_OK;
}
#undef TIMED

// Capture `steps` consecutive decode steps as one graph.
int capture_steps(ptmi_model *m, int steps, hipGraph_t *graph_out, hipGraphExec_t *exec_out) {
    hipStream_t s = lib_stream();
    PTMI_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int st = PTMI_OK;
    for (int i = 0; i < steps && st == PTMI_OK; i++) st = enqueue_step(m, s);
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(s, &graph);
    if (st) { if (graph) (void)hipGraphDestroy(graph); return st; }
    if (e != hipSuccess) return hip_check(e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) { (void)hipGraphDestroy(graph); return hip_check(e, "hipGraphInstantiate"); }
    *graph_out = graph;
    *exec_out = exec;
    return PTMI_OK;
}

int build_graph(ptmi_model *m) {
    int st = capture_steps(m, 1, &m->graph, &m->exec);
    if (st == PTMI_OK && m->graph_steps > 1) st = capture_steps(m, m->graph_steps, &m->graph_k, &m->exec_k);
    return st;
}

// One decode step: the captured graph, or the same launches enqueued
// directly when PTMI_DECODE_EAGER=1 (profilers that do not follow graph
// launches).
int launch_step(ptmi_model *m, hipStream_t s) {
    if (m->eager) return enqueue_step(m, s);
    PTMI_HIP(hipGraphLaunch(m->exec, s));
    return PTMI_OK;
}

// n consecutive decode steps: graphs of graph_steps steps while enough
// remain, then single steps.
int launch_steps(ptmi_model *m, hipStream_t s, int n) {
    int st;
    if (!m->eager && m->exec_k)
        for (; n >= m->graph_steps; n -= m->graph_steps) PTMI_HIP(hipGraphLaunch(m->exec_k, s));
    for (; n > 0; n--)
        if ((st = launch_step(m, s))) return st;
    return PTMI_OK;
}

// The host's four fields of the control block (the step sequence number
// and the error word stay as the device left them).
int set_ctl(ptmi_model *m, int tok, int pos, int n_prompt) {
    const int h[4] = {tok, pos, n_prompt, 0};
    PTMI_HIP(hipMemcpyAsync(m->ctl, h, sizeof(h), hipMemcpyHostToDevice, lib_stream()));
    return PTMI_OK;
}

// After a synchronised step: a wait of the one-kernel step that timed out
// is an error (the step's results are void).  The error word is cleared and
// the step sequence number moved past the failed step's, whose partly
// written exchange words carry its tag and must never match a later step.
int check_step_error(ptmi_model *m, const DecodeCtl &h) {
    if (!h.err) return PTMI_OK;
    const int fix[2] = {h.seq + 1, 0};                   // seq, err
    PTMI_HIP(hipMemcpy(&m->ctl->seq, fix, sizeof(fix), hipMemcpyHostToDevice));
    return set_error(PTMI_ERR_STATE, "decode step: a workgroup timed out waiting for another's results");
}

int zero_kv(ptmi_model *m) {
    const size_t n = (size_t)m->c.n_layers * m->c.seq_len * m->c.kv_dim * sizeof(float);
    PTMI_HIP(hipMemsetAsync(m->kc, 0, n, lib_stream()));
    PTMI_HIP(hipMemsetAsync(m->vc, 0, n, lib_stream()));
    return PTMI_OK;
}

}  // namespace

}  // namespace ptmi

using namespace ptmi;

extern "C" {

int ptmi_model_create(const void *blob, size_t bytes, int max_T, ptmi_model_t **out) {
    if (!out) return set_error(PTMI_ERR_ARG, "ptmi_model_create: out is NULL");
    *out = nullptr;
    int st = PTMI_OK;
    // The model holds the blob's registration until ptmi_model_destroy;
    // every failure below releases it again.
    Resident *r = register_blob(blob, bytes, false, &st);
    if (!r) return st;
    const Config &c = r->c;
    if (c.dim % 4 || c.hidden % 4 || c.head_dim % 4 || c.head_dim > kMaxHeadDim || c.seq_len > kMaxSeqLen ||
        c.dim > kMaxCombineDim) {
        st = set_error(PTMI_ERR_ARG, "unsupported shape: dim=%d hidden=%d head_dim=%d", c.dim, c.hidden,
                       c.head_dim);
        release_blob(r);
        return st;
    }
    // Grouped-query attention is refused: the reference's rope() rotates k
    // over dim floats (pt_ops.c:33-49, called at llama2.c:147) while s->k
    // holds kv_dim floats (llama2.c:81), so it has no defined result to
    // match there, and no configuration uses it.
    if (c.n_kv_heads != c.n_heads) {
        st = set_error(PTMI_ERR_ARG, "n_kv_heads=%d != n_heads=%d: grouped-query attention is not supported",
                       c.n_kv_heads, c.n_heads);
        release_blob(r);
        return st;
    }
    if (max_T < 0 || max_T > c.seq_len) {
        st = set_error(PTMI_ERR_ARG, "max_T=%d outside [0, seq_len]", max_T);
        release_blob(r);
        return st;
    }
    ptmi_model *m = new ptmi_model();
    m->res = r;
    m->c = c;
    m->max_T = max_T;
    const size_t D = c.dim, H = c.hidden, V = c.vocab, S = c.seq_len, KV = c.kv_dim, L = c.n_layers;
    // attention chunks: <= 8 per head, 64..kMaxAttnChunk positions each
    // (seq_len 1024: 128; 64- and 256-position chunks measured slower, the
    // first by its costlier combine, the second by its longer streams)
    const int per = (c.seq_len + 7) / 8;
    m->attn_chunk = std::min(kMaxAttnChunk, std::max(64, (per + 63) / 64 * 64));
    m->attn_chunks = (c.seq_len + m->attn_chunk - 1) / m->attn_chunk;
    const size_t NH = c.n_heads, NC = m->attn_chunks, hd = c.head_dim;
    size_t sizes[] = {D, D, D, H, V, L * S * KV, L * S * KV, NH * NC * hd, NH * NC * 2};
    float **dst[] = {&m->x, &m->xb, &m->q, &m->hb, &m->logits, &m->kc, &m->vc, &m->part_o, &m->part_ml};
    size_t total = 0;
    for (size_t s : sizes) total += align_up(s, 64);
    const size_t ints = align_up(sizeof(DecodeCtl) / 4, 64) + 2 * align_up(S, 64) + 64;
    total += ints;
    hipError_t e = hipMalloc(&m->mem, total * sizeof(float));
    if (e != hipSuccess) {
        st = hip_check(e, "hipMalloc(decode state)");
        delete m;
        release_blob(r);
        return st;
    }
    size_t o = 0;
    for (int i = 0; i < 9; i++) { *dst[i] = m->mem + o; o += align_up(sizes[i], 64); }
    m->ctl = (DecodeCtl *)(m->mem + o); o += align_up(sizeof(DecodeCtl) / 4, 64);
    m->prompt = (int *)(m->mem + o); o += align_up(S, 64);
    m->out_tokens = (int *)(m->mem + o); o += align_up(S, 64);
    m->sink = m->mem + o;
    hipStream_t s = lib_stream();
    e = hipMemsetAsync(m->mem, 0, total * sizeof(float), s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        st = hip_check(e, "zero decode state");
        (void)hipFree(m->mem);
        delete m;
        release_blob(r);
        return st;
    }
    const char *eager = getenv("PTMI_DECODE_EAGER");
    m->eager = eager && eager[0] == '1';
    if (const char *gs = getenv("PTMI_DECODE_GRAPH_STEPS")) m->graph_steps = std::max(1, std::min(64, atoi(gs)));
    const char *nopf = getenv("PTMI_NO_PREFETCH");
    m->prefetch = !(nopf && nopf[0] == '1');
    if (const char *pp = getenv("PTMI_PREFETCH_PLAN")) {
        if (strlen(pp) != 7 || strspn(pp, "ofdqOF-") != 7) {
            st = set_error(PTMI_ERR_ARG, "PTMI_PREFETCH_PLAN: 7 letters of ofdqOF- expected, got \"%s\"", pp);
            (void)hipFree(m->mem);
            delete m;
            release_blob(r);
            return st;
        }
        memcpy(m->prefetch_plan, pp, 8);
    }
    if ((st = decode_step_create(m)) || (!m->eager && (st = build_graph(m))) ||
        (max_T > 0 && (st = train_create(m)))) {
        train_destroy(m);
        decode_step_destroy(m);
        if (m->exec) (void)hipGraphExecDestroy(m->exec);
        if (m->graph) (void)hipGraphDestroy(m->graph);
        if (m->exec_k) (void)hipGraphExecDestroy(m->exec_k);
        if (m->graph_k) (void)hipGraphDestroy(m->graph_k);
        (void)hipFree(m->mem);
        delete m;
        release_blob(r);
        return st;
    }
    *out = m;
    return PTMI_OK;
}

void ptmi_model_destroy(ptmi_model_t *m) {
    if (!m) return;
    (void)hipStreamSynchronize(lib_stream());
    train_destroy(m);
    if (m->exec) (void)hipGraphExecDestroy(m->exec);
    if (m->graph) (void)hipGraphDestroy(m->graph);
    if (m->exec_k) (void)hipGraphExecDestroy(m->exec_k);
    if (m->graph_k) (void)hipGraphDestroy(m->graph_k);
    decode_step_destroy(m);
    (void)hipFree(m->mem);
    release_blob(m->res);
    delete m;
}

int ptmi_model_config(const ptmi_model_t *m, int cfg7[7]) {
    if (!m || !cfg7) return set_error(PTMI_ERR_ARG, "ptmi_model_config: NULL");
    const Config &c = m->c;
    int v[7] = {c.dim, c.hidden, c.n_layers, c.n_heads, c.n_kv_heads, c.vocab, c.seq_len};
    memcpy(cfg7, v, sizeof(v));
    return PTMI_OK;
}

int ptmi_model_reset_kv(ptmi_model_t *m) {
    if (!m) return set_error(PTMI_ERR_ARG, "NULL model");
    int st;
    if ((st = zero_kv(m)) || (st = set_ctl(m, 0, 0, 0))) return st;
    PTMI_HIP(hipStreamSynchronize(lib_stream()));
    m->host_pos = 0;
    return PTMI_OK;
}

int ptmi_model_pos(const ptmi_model_t *m) { return m ? m->host_pos : -1; }

int ptmi_model_forward_step(ptmi_model_t *m, int token, int *next) {
    if (!m) return set_error(PTMI_ERR_ARG, "NULL model");
    if (token < 0 || token >= m->c.vocab) return set_error(PTMI_ERR_ARG, "token %d outside [0, %d)", token, m->c.vocab);
    if (m->host_pos >= m->c.seq_len)
        return set_error(PTMI_ERR_STATE, "position %d: KV cache full (seq_len %d)", m->host_pos, m->c.seq_len);
    hipStream_t s = lib_stream();
    int st;
    if ((st = set_ctl(m, token, m->host_pos, 0)) || (st = launch_step(m, s))) return st;
    DecodeCtl h;
    PTMI_HIP(hipMemcpyAsync(&h, m->ctl, sizeof(h), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    if ((st = check_step_error(m, h))) return st;
    m->host_pos++;
    if (next) *next = h.next;
    return PTMI_OK;
}

int ptmi_model_logits(ptmi_model_t *m, float *out) {
    if (!m || !out) return set_error(PTMI_ERR_ARG, "NULL argument");
    hipStream_t s = lib_stream();
    PTMI_HIP(hipMemcpyAsync(out, m->logits, (size_t)m->c.vocab * sizeof(float), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    return PTMI_OK;
}

int ptmi_model_generate(ptmi_model_t *m, const int *prompt, int n_prompt, int max_tokens, int stop_on_eos,
                        int *out, int *n_out) {
    if (!m || !prompt || !out || !n_out || n_prompt < 1)
        return set_error(PTMI_ERR_ARG, "ptmi_model_generate: bad arguments");
    const Config &c = m->c;
    if (max_tokens > c.seq_len) max_tokens = c.seq_len;          // pt_text.c:321-322
    if (n_prompt > c.seq_len) return set_error(PTMI_ERR_ARG, "prompt longer than seq_len");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= c.vocab) return set_error(PTMI_ERR_ARG, "prompt[%d]=%d out of range", i, prompt[i]);
    *n_out = 0;
    if (max_tokens <= 0) return PTMI_OK;
    hipStream_t s = lib_stream();
    int st;
    if ((st = zero_kv(m))) return st;
    PTMI_HIP(hipMemcpyAsync(m->prompt, prompt, (size_t)n_prompt * sizeof(int), hipMemcpyHostToDevice, s));
    if ((st = set_ctl(m, prompt[0], 0, n_prompt))) return st;
    if ((st = launch_steps(m, s, max_tokens))) return st;
    PTMI_HIP(hipMemcpyAsync(out, m->out_tokens, (size_t)max_tokens * sizeof(int), hipMemcpyDeviceToHost, s));
    DecodeCtl h;
    PTMI_HIP(hipMemcpyAsync(&h, m->ctl, sizeof(h), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    if ((st = check_step_error(m, h))) return st;
    m->host_pos = max_tokens;
    int n = max_tokens;
    if (stop_on_eos)                                               // pt_text.c:354
        for (int i = n_prompt - 1; i < max_tokens; i++)
            if (out[i] == 1 || out[i] == 2) { n = i + 1; break; }
    *n_out = n;
    return PTMI_OK;
}

int ptmi_model_decode_async(ptmi_model_t *m, int first_token, int n_steps) {
    if (!m) return set_error(PTMI_ERR_ARG, "NULL model");
    if (first_token < 0 || first_token >= m->c.vocab) return set_error(PTMI_ERR_ARG, "token out of range");
    if (n_steps < 0 || m->host_pos + n_steps > m->c.seq_len)
        return set_error(PTMI_ERR_STATE, "pos %d + %d steps exceeds seq_len %d", m->host_pos, n_steps, m->c.seq_len);
    hipStream_t s = lib_stream();
    int st;
    if ((st = set_ctl(m, first_token, m->host_pos, 0))) return st;
    if ((st = launch_steps(m, s, n_steps))) return st;
    m->host_pos += n_steps;
    return PTMI_OK;
}

int ptmi_model_sync(ptmi_model_t *m) {
    if (!m) return set_error(PTMI_ERR_ARG, "NULL model");
    hipStream_t s = lib_stream();
    DecodeCtl h;
    PTMI_HIP(hipMemcpyAsync(&h, m->ctl, sizeof(h), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    return check_step_error(m, h);
}

int ptmi_model_profile(ptmi_model_t *m, int first_token, int n_steps, float role_ms[8], int role_launches[8]) {
    if (!m || !role_ms || !role_launches) return set_error(PTMI_ERR_ARG, "NULL argument");
    if (first_token < 0 || first_token >= m->c.vocab) return set_error(PTMI_ERR_ARG, "token out of range");
    if (n_steps < 0 || m->host_pos + n_steps > m->c.seq_len)
        return set_error(PTMI_ERR_STATE, "pos %d + %d steps exceeds seq_len %d", m->host_pos, n_steps, m->c.seq_len);
    for (int i = 0; i < 8; i++) { role_ms[i] = 0.0f; role_launches[i] = 0; }
    hipStream_t s = lib_stream();
    int st;
    if ((st = set_ctl(m, first_token, m->host_pos, 0))) return st;
    StepTimer tm;
    for (int k = 0; k < n_steps; k++) {
        tm.used = 0;
        if ((st = enqueue_step(m, s, &tm))) return st;
        PTMI_HIP(hipStreamSynchronize(s));
        DecodeCtl h;
        PTMI_HIP(hipMemcpy(&h, m->ctl, sizeof(h), hipMemcpyDeviceToHost));
        if ((st = check_step_error(m, h))) return st;
        for (size_t i = 0; i < tm.used / 2; i++) {
            float ms = 0.0f;
            PTMI_HIP(hipEventElapsedTime(&ms, tm.ev[2 * i], tm.ev[2 * i + 1]));
            role_ms[tm.role[i]] += ms;
            role_launches[tm.role[i]]++;
        }
        m->host_pos++;
    }
    return PTMI_OK;
}

int ptmi_model_read_weights(ptmi_model_t *m, void *blob, size_t bytes) {
    if (!m || !blob) return set_error(PTMI_ERR_ARG, "NULL argument");
    if (bytes < m->res->bytes) return set_error(PTMI_ERR_ARG, "destination smaller than the blob");
    if (blob != (void *)m->res->blob) memcpy(blob, m->res->blob, m->res->bytes);   // header, freq_cis
    return download_resident(m->res, blob, lib_stream());
}

}  // extern "C"
