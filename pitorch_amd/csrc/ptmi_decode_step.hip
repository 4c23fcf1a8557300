// The decode step (pt_forward_step over pt_forward, pitorch/model/llama2.c:
// 127-206, plus the argmax of pitorch/pt.c:267-271) as ONE persistent
// kernel launch per token.
//
// A kernel boundary on this part costs ~4 us per dependent stage (launch,
// L2 invalidate, then the first weight round trip); the step has 5L+2 such
// stages.  Here every workgroup walks all stages of the token:
//  * each stage's weights are loaded into registers BEFORE the workgroup
//    waits for the stage's input, so the weight stream overlaps the
//    dependency latency instead of following it;
//  * every value handed between workgroups within the token is one 64-bit
//    word (float bits | 32-bit tag), written and read with agent-scope
//    relaxed atomics (they bypass the per-XCD L2s, which are not coherent
//    with each other).  The tag is the step's sequence number, so a reader
//    never accepts a value of an earlier token, and every (layer, stage)
//    has its own buffer, so nothing is overwritten while it can still be
//    read.  A consumer polls exactly the words it needs — no barrier
//    flags, no fences.
//  * data that only later tokens read (the KV cache rows of this position)
//    and the logits the host reads are plain stores: the kernel boundary
//    between tokens makes them visible.
// Every wait is bounded (20 ms of the 100 MHz real-time counter) and
// checks a shared error word, so on any failure every wave leaves within
// one bound and the host reports the error.
//
// Stages per layer (workgroup b takes row blocks b, b+NB, ...):
//   QKV  : RMSNorm(x) . [Wq;Wk;Wv], RoPE, q|k|v published, K/V cache row
//   ATT  : (head, chunk of positions) units: scores, chunk softmax, e.v;
//          the head's chunk-0 unit merges the chunks           -> att
//   WO   : att . Wo, + residual                                -> x_a
//   W13  : RMSNorm(x_a) . [w1|w3] rows interleaved, SwiGLU     -> hb
//   W2   : hb . w2 + x_a                                         -> x_b
// then the classifier (RMSNorm . Wcls, per-workgroup argmax candidates)
// and workgroup 0's final argmax, prompt forcing and position advance.
// Arithmetic per element follows the multi-kernel step (and through it
// the reference's ops); reductions run in a different order.
#include "ptmi_model.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>

namespace ptmi {

namespace {

constexpr int kT = 512;                      // threads per workgroup
constexpr int kW = kT / 64;                  // waves per workgroup
constexpr int kRowsD = 2 * kW;               // rows per block, D-length rows (32 lanes per row)
constexpr int kRowsH = kW;                   // rows per block, H-length rows (64 lanes per row)
constexpr int kAttRows = 128;                // attention positions per unit (at most)
constexpr int kMaxChunks = 8;                // units per head
// Copies of the w1|w3 stage input x_a (Wo's output), in kRepXa regions of
// L*D tagged words.  Every workgroup polls the whole vector at once, and
// workgroup b polls copy b % kRepXa: the chip's workgroups are dealt to its 8
// XCDs in turn, so each copy's lines are read from one XCD.  Same box,
// stories110M tok/s: one copy 6070-6080, 4 copies 6133-6136, 8 copies
// 6156-6171, 16 copies 6071-6073.  Copies of x_b (the next QKV and the
// classifier input) or of the hidden vector were slower: the storing waves
// wait for their extra stores before their next poll.
constexpr int kRepXa = 8;
// w2's waves store their own rows (no barrier) on the instantiations with
// 6 float4 per lane of a dim row (dim 768), and the copies of x_b that the
// other instantiations store after w2's barrier (kernel and host agree
// through these two functions).
constexpr bool w2_direct(int itd) { return itd >= 6; }
constexpr int rep_xb(int itd) { return w2_direct(itd) ? 1 : kW; }
constexpr int kWriter = kW - 1;              // the wave that issues the workgroup's global stores (not w1|w3's or w2's)
constexpr int kPollT = kWriter * 64;         // threads that poll (all other waves)
constexpr int kMaxHd = 64;                   // head_dim of the instantiated kernels (16 lanes x float4)
constexpr int kPartLds = kMaxChunks * (kMaxHd + 2);  // floats of one head's chunk records
constexpr uint64_t kWaitTicks = 2000000;     // default wait bound: 20 ms at 100 MHz

typedef float fx4 __attribute__((ext_vector_type(4)));

struct StepArgs {
    // weights (device layout of the registered blob)
    const float *emb, *rms_att, *wqkv, *wo, *rms_ffn, *w13, *w2, *rms_final, *wcls;
    int D, H, L, NH, KV, hd, kv_mul, V, S;
    int chunk, n_chunks;                     // attention unit = chunk positions of one head
    int ubase;                               // workgroup of attention unit 0
    int qbase;                               // workgroup of QKV row block 0
    int wbase;                               // workgroup of Wo row block 0 (a QKV workgroup)
    float att_scale;
    float *kc, *vc;                          // [L][S][KV]
    float *logits;                           // [V]
    DecodeCtl *ctl;
    const int *prompt;
    int *out_tokens;
    // tagged exchange buffers: word = tag << 32 | float bits
    uint64_t *t_qkv;                         // [L][D + 2KV]
    uint64_t *t_part;                        // [L][NH][n_chunks][hd + 2]  (o[hd], max, sum)
    uint64_t *t_att;                         // [L][D]  merged attention output per head
    uint64_t *t_xa, *t_xb;                   // [kRepXa][L][D], [rep_xb(itd)][L][D]
    uint64_t *t_hb;                          // [L][H]
    uint64_t *t_cand;                        // [nb][2]  (best logit, its index)
    // optional stage stamps (PTMI_STEP_STAMPS=1): per workgroup, the 100 MHz
    // real-time counter at kernel start, then for every stage the end of
    // its wait and the end of its work; 0 where the workgroup had no part
    uint64_t *stamps;                        // [nb][n_stamps]
    int n_stamps;                            // 1 + 10 L + 4
    uint64_t wait_ticks;                     // bound of every wait (100 MHz ticks)
    int l2pf;                                // L2 staging by idle workgroups: 1 w1|w3 + w2, 2 next QKV + Wo
    int cls_pf;                              // classifier row blocks each w2-idle workgroup stages in the last layer
    int poison;                              // test only: chunk-record LDS starts as NaN (PTMI_STEP_POISON_LDS=1)
};


// Every pointer of the argument block points to global memory; accesses
// go through the global address space explicitly (pointers read from
// memory are otherwise generic, and flat instructions also count against
// the LDS counter, so an LDS read would wait for every flat load in flight).
#define PTMI_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ PTMI_GLOBAL T *gl(T *p) {
    return (PTMI_GLOBAL T *)p;
}

// The argument block is read through the constant address space: its
// fields come in with scalar loads.
#define PTMI_CONST __attribute__((address_space(4)))

// Stamp slot `i` of this workgroup (one thread of the writer wave; no-op
// without stamps).  Stamps collect in LDS and reach global memory only as
// the workgroup leaves (flush_stamps): a global store here would sit in the
// wave's memory counter and delay its next wait.
constexpr int kStampSlots = 1 + 10 * 32 + 4;       // up to 32 layers
__device__ __forceinline__ void stamp(const PTMI_CONST StepArgs *a, uint64_t *st, int i) {
    if (a->stamps && threadIdx.x == kPollT) st[i] = __builtin_amdgcn_s_memrealtime();
}
// The writer wave copies this launch's stamps (the non-zero slots) out.
__device__ __forceinline__ void flush_stamps(const PTMI_CONST StepArgs *a, const uint64_t *st) {
    if (!a->stamps || ((int)threadIdx.x >> 6) != kWriter) return;
    for (int i = (int)threadIdx.x & 63; i < a->n_stamps; i += 64)
        if (st[i]) gl(a->stamps)[(long)blockIdx.x * a->n_stamps + i] = st[i];
}

__device__ __forceinline__ uint64_t tload(const uint64_t *p) {
    return __hip_atomic_load(gl(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(uint64_t *p, float v, uint32_t tag) {
    __hip_atomic_store(gl(p), ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int err_seen(const DecodeCtl *c) {
    return __hip_atomic_load(gl(&c->err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A value the compiler cannot see through: per-thread addresses derived
// from it are recomputed where they are used (a few ALU operations)
// instead of being hoisted out of the layer loop and held in registers
// for the whole kernel.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float4 sel4(bool keep, float4 v) {
    return make_float4(keep ? v.x : 0.0f, keep ? v.y : 0.0f, keep ? v.z : 0.0f, keep ? v.w : 0.0f);
}
__device__ __forceinline__ float dot4(float4 a, float4 b, float acc) {
    acc = fmaf(a.x, b.x, acc);
    acc = fmaf(a.y, b.y, acc);
    acc = fmaf(a.z, b.z, acc);
    return fmaf(a.w, b.w, acc);
}
__device__ __forceinline__ float4 load4(const float *p) {
    const fx4 t = *gl(reinterpret_cast<const fx4 *>(p));
    return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ float4 ntload4(const float *p) {
    const fx4 t = __builtin_nontemporal_load(gl(reinterpret_cast<const fx4 *>(p)));
    return make_float4(t.x, t.y, t.z, t.w);
}

// Wait until the n tagged words of src carry `tag`; their values go to
// dst (LDS).  The calling thread takes words t, t + kPollT, ... (t = its
// index among the callers), at most K of them, and re-reads only those
// still missing.  Returns false on a timeout or when another workgroup has
// already failed.
// Only waves other than the writer wave poll: on this GPU a wave's loads
// and stores share one in-order counter, so a wave that has just stored
// would see its poll wait for the acknowledgement of its stores.
// The shared error word is a single line that every waiting thread of the
// chip would read on every round; it is read every 32nd round only.
template <int K>
__device__ bool poll_words(const uint64_t *src, int n, uint32_t tag, float *dst, const PTMI_CONST StepArgs *a, int t) {
    t = opaque(t);
    bool ok[K];
#pragma unroll
    for (int k = 0; k < K; k++) ok[k] = t + k * kPollT >= n;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    const uint64_t wait_ticks = a->wait_ticks;
    for (int round = 1;; round++) {
        uint64_t v[K];
#pragma unroll
        for (int k = 0; k < K; k++)
            if (!ok[k]) v[k] = tload(src + t + k * kPollT);
        bool all = true;
#pragma unroll
        for (int k = 0; k < K; k++) {
            if (ok[k]) continue;
            if ((uint32_t)(v[k] >> 32) == tag) {
                dst[t + k * kPollT] = __uint_as_float((uint32_t)v[k]);
                ok[k] = true;
            } else {
                all = false;
            }
        }
        if (all) return true;
        if (__builtin_amdgcn_s_memrealtime() - t0 > wait_ticks) return false;
        if ((round & 31) == 0 && err_seen(a->ctl)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

// poll_words over word pairs: one 16-byte load (coherent at system scope,
// so it bypasses the XCD's L2 like the agent-scope loads) brings two tagged
// words, half the load requests of poll_words for a long vector.  Pair p of thread t is words 2p, 2p+1, p = t, t + kPollT, ...;
// src must be 16-byte aligned and n even.
typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSysScope = 1 | 16;            // buffer cache policy: sc0 | sc1
template <int K, int NT = kPollT>
__device__ bool poll_pairs(const uint64_t *src, int n, uint32_t tag, float *dst, const PTMI_CONST StepArgs *a, int t) {
    t = opaque(t);
    const int np = n >> 1;
    bool valid[K], ok[K];
#pragma unroll
    for (int k = 0; k < K; k++) ok[k] = !(valid[k] = t + k * NT < np);
    // every round loads all K pairs (past the vector: its last pair again),
    // so each register set is only ever written by a load.  The loads are
    // buffer loads with the system-scope cache bits (sc0 sc1: past this
    // XCD's L2, like a volatile load) but not volatile: a volatile load is
    // followed by a wait for it, which would serialise a round's loads and
    // the two rounds.  The offset goes through opaque() at every load, so no
    // load is taken as loop-invariant.
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)src, (short)0, np * 16, 0x00020000);
    auto pair = [&](int k) {
        const u32x4 w = __builtin_amdgcn_raw_buffer_load_b128(rs, opaque(16 * min(t + k * NT, np - 1)), 0, kSysScope);
        u64x2 v;
        v.x = (uint64_t)w.x | ((uint64_t)w.y << 32);
        v.y = (uint64_t)w.z | ((uint64_t)w.w << 32);
        return v;
    };
    // Two rounds in flight: round r + 1's loads go out before round r's
    // words are checked, so a word that lands is seen about half a round
    // trip sooner than with one round at a time.  The loop alternates two
    // register sets (a copy between them would wait for the loads).
    u64x2 va[K], vb[K];
#pragma unroll
    for (int k = 0; k < K; k++) va[k] = pair(k);
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    const uint64_t wait_ticks = a->wait_ticks;
    auto check = [&](const u64x2 (&v)[K]) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < K; k++) {
            if (ok[k]) continue;
            if ((uint32_t)(v[k].x >> 32) == tag && (uint32_t)(v[k].y >> 32) == tag) {
                const int i = 2 * (t + k * NT);
                dst[i] = __uint_as_float((uint32_t)v[k].x);
                dst[i + 1] = __uint_as_float((uint32_t)v[k].y);
                ok[k] = true;
            } else {
                all = false;
            }
        }
        return all;
    };
    // The wave leaves the loop together (a lane that has all its words
    // keeps loading until every lane has): with per-lane exits the loop's
    // register sets are copied at its latch, which waits for their loads.
    asm volatile("" ::: "memory");
    for (int round = 1;; round += 2) {
#pragma unroll
        for (int k = 0; k < K; k++) vb[k] = pair(k);
        asm volatile("" ::: "memory");
        if (__all(check(va))) return true;
        if (__builtin_amdgcn_s_memrealtime() - t0 > wait_ticks) return false;
        if ((round & 31) == 1 && __any(err_seen(a->ctl))) return false;
#pragma unroll
        for (int k = 0; k < K; k++) va[k] = pair(k);
        asm volatile("" ::: "memory");
        if (__all(check(vb))) return true;
    }
}

// Block-uniform end of a wait: every thread reaches the barrier; true when
// the whole block may go on.
__device__ __forceinline__ bool block_ok(bool mine, int *s_fail, DecodeCtl *ctl) {
    if (!mine) {
        *s_fail = 1;
        __hip_atomic_fetch_or(gl(&ctl->err), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *s_fail == 0;
}

// argmax pair (value, index): larger value, ties to the smaller index
// (pt_ops.c:65-70 returns the first index of the maximum).
__device__ __forceinline__ void take_best(float &bv, int &bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

// The argument block lives in device memory; every stage re-reads the
// fields it needs through a pointer the compiler cannot see through, so
// uniform values are reloaded per stage (scalar-cache hits) instead of
// being held in scalar registers across the whole layer loop.
__device__ __forceinline__ const PTMI_CONST StepArgs *fresh(const StepArgs *p) {
    asm volatile("" : "+s"(p));
    return (const PTMI_CONST StepArgs *)p;
}

// Per-token values read once at kernel start.
struct Tok {
    int pos, token, nact;
    uint32_t tag;
};

// Workgroup LDS.
struct Smem {
    float xs[2048];                    // the stage's input vector (<= max(D, H))
    float part[kPartLds];              // ATT, chunk 0: the head's chunk records
    float xres[kRowsD];                // WO: residual rows of this block
    float xres2[kRowsH];               // W2: residual rows of this block
    float rope_c[64], rope_s[64];      // RoPE cos/sin of this position, pair i = 2*k (all layers)
    int rope_k[kRowsD];                // QKV: the RoPE pair of each row of this workgroup's first block
    float ybuf[kW][2];                 // argmax per wave
    float qs[128], kp[128], vp[128];   // ATT: q, and k/v of this position
    float mrg[kMaxHd];                 // ATT, chunk 0: the merged head output
    float red[kW][128];
    float wred[kW];
    float sc[kAttRows];                // ATT: scores -> weights
    float wred2[kW];                   // ATT: per-wave sums of e^(s - max)
    float cand[1024];                  // final argmax: (value, index) per workgroup
    float yout[kRowsD];                // results the writer wave stores
    uint64_t st[kStampSlots];          // stage stamps until the workgroup leaves
    float ycls[2][kRowsD];             // classifier logits, alternate row blocks
    int fail;
};

// Per-lane registers carried between stages: the weights of the next
// stage (loaded before its wait) and the K/V rows of the attention unit.
template <int ITD, int ITH, int GA>
struct Regs {
    static constexpr int kRPW = 64 / GA;                 // K/V rows per wave load
    static constexpr int kU = kAttRows / (kW * kRPW);    // loads per thread per chunk
    float4 wD[ITD], nw[ITD], wH[ITH];
    float4 kk[kU], vv[kU];
};

__device__ __forceinline__ int slot_d() { return opaque(((int)threadIdx.x >> 6) * 2 + (((int)threadIdx.x & 63) >> 5)); }
__device__ __forceinline__ int sub_d() { return opaque((int)threadIdx.x & 31); }

// Weights of D-length row block rb of W (rows x D) and, when norm is set,
// the RMSNorm weights of this lane's columns.  Rows past the matrix
// re-read its last row; chunks past the row re-read its last chunk (both
// dropped at use).
template <int ITD, int ITH, int GA>
__device__ __forceinline__ void load_wD(const PTMI_CONST StepArgs *a, Regs<ITD, ITH, GA> &R, const float *W, int rows, int rb,
                                        const float *norm) {
    const int nD4 = a->D >> 2, slot = slot_d(), sub = sub_d();
    const int r = min(rb * kRowsD + slot, rows - 1);
    const float *row = W + (long)r * a->D;
#pragma unroll
    for (int it = 0; it < ITD; it++) R.wD[it] = ntload4(row + 4 * min(sub + it * 32, nD4 - 1));
    if (norm) {
#pragma unroll
        for (int it = 0; it < ITD; it++) R.nw[it] = load4(norm + 4 * min(sub + it * 32, nD4 - 1));
    }
}

template <int ITD, int ITH, int GA>
__device__ __forceinline__ void load_wH(const PTMI_CONST StepArgs *a, Regs<ITD, ITH, GA> &R, const float *W, int rows, int rb) {
    const int nH4 = a->H >> 2, slot = opaque((int)threadIdx.x >> 6), sub = opaque((int)threadIdx.x & 63);
    const int r = min(rb * kRowsH + slot, rows - 1);
    const float *row = W + (long)r * a->H;
#pragma unroll
    for (int it = 0; it < ITH; it++) R.wH[it] = ntload4(row + 4 * min(sub + it * 64, nH4 - 1));
}

// Wo rows are D-length rows like the QKV and w1|w3 rows (same lane layout),
// held in the first ITD registers of the w2 set: it is free from the w2 dot
// to the next layer's Wo dot, so a workgroup can hold the Wo rows and the
// w1|w3 rows at once.
template <int ITD, int ITH, int GA>
__device__ __forceinline__ void load_wo(const PTMI_CONST StepArgs *a, Regs<ITD, ITH, GA> &R, int l, int rb) {
    static_assert(ITH >= ITD, "the Wo rows live in the w2 registers");
    const int D = a->D, nD4 = D >> 2, sub = sub_d();
    const float *row = a->wo + (long)l * D * D + (long)min(rb * kRowsD + slot_d(), D - 1) * D;
#pragma unroll
    for (int it = 0; it < ITD; it++) R.wH[it] = ntload4(row + 4 * min(sub + it * 32, nD4 - 1));
}
// The lane's chunks of the stage input xs (LDS), all reads issued before
// any is used: one wait for the batch instead of one LDS round trip per
// chunk (the scheduler otherwise interleaves each read with its use).
template <int N, int STRIDE>
__device__ __forceinline__ void read_xs(const float *xs, int n4, int sub, float4 (&xr)[N]) {
#pragma unroll
    for (int it = 0; it < N; it++) {
        const int c = sub + it * STRIDE;
        xr[it] = reinterpret_cast<const float4 *>(xs)[min(c, n4 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    if (n4 < N * STRIDE) {                            // uniform: rows shorter than the lanes' span
#pragma unroll
        for (int it = 0; it < N; it++) xr[it] = sel4(sub + it * STRIDE < n4, xr[it]);
    }
}

// sum over the lane's chunks of w . x; chunks past the row (clamped
// re-reads) are dropped, and a row that fills every lane's chunks takes the
// branch without the selects (the same sums)
template <int N, int STRIDE>
__device__ __forceinline__ float dot_chunks(const float4 (&w)[N], const float4 (&x)[N], int n4, int sub) {
    float acc = 0.0f;
    if (n4 >= N * STRIDE) {                           // uniform
#pragma unroll
        for (int it = 0; it < N; it++) acc = dot4(w[it], x[it], acc);
    } else {
#pragma unroll
        for (int it = 0; it < N; it++) acc = dot4(sel4(sub + it * STRIDE < n4, w[it]), x[it], acc);
    }
    return acc;
}

template <int ITD, int ITH, int GA>
__device__ __forceinline__ float dot_wo(const PTMI_CONST StepArgs *a, const Regs<ITD, ITH, GA> &R, const float *xs) {
    const int nD4 = a->D >> 2, sub = sub_d();
    float4 xr[ITD];
    read_xs<ITD, 32>(xs, nD4, sub, xr);
    float4 wr[ITD];
#pragma unroll
    for (int it = 0; it < ITD; it++) wr[it] = R.wH[it];
    return group_sum<32>(dot_chunks<ITD, 32>(wr, xr, nD4, sub));
}

// 1/sqrt(v) of an RMSNorm (pt_ops.c:9: 1 / pt_sqrtf(ss / dim + 1e-5)) as
// the hardware reciprocal square root: one instruction (about 1 ulp) in
// place of the reference's three Newton steps of IEEE divisions and a
// fourth division, which were the longest dependent chain of the QKV and
// w1|w3 stages (5548 -> 5771 tok/s, same box; greedy tokens identical).
__device__ __forceinline__ float rms_inv(float v) { return __builtin_amdgcn_rsqf(v); }

// The lane's D-row weights against xs (RMSNorm'd when norm): the row's sum
// in every lane of its 32-lane group.
template <int ITD, int ITH, int GA>
__device__ __forceinline__ float dot_d(const PTMI_CONST StepArgs *a, const Regs<ITD, ITH, GA> &R, const float *xs, bool norm) {
    const int nD4 = a->D >> 2, sub = sub_d();
    float4 xr[ITD];
    read_xs<ITD, 32>(xs, nD4, sub, xr);
    if (norm) {
        // rmsnorm (pt_ops.c:5-12) with its scalar factored out of the dot:
        // y = inv * sum_j W_j (w_j x_j).  The sum of squares, its sqrt and
        // the division no longer precede the dot, they run beside it
        // (independent chains), and the 1/rms scale is one multiply at the
        // end; per output one rounding moves (inv applied to the sum, not to
        // each x_j), within the matvec tolerance.
        float ss = 0.0f;
#pragma unroll
        for (int it = 0; it < ITD; it++)
            ss = dot4(xr[it], xr[it], ss);
        float4 xg[ITD];
#pragma unroll
        for (int it = 0; it < ITD; it++) {
            xg[it].x = xr[it].x * R.nw[it].x;
            xg[it].y = xr[it].y * R.nw[it].y;
            xg[it].z = xr[it].z * R.nw[it].z;
            xg[it].w = xr[it].w * R.nw[it].w;
        }
        float raw = dot_chunks<ITD, 32>(R.wD, xg, nD4, sub);
        ss = group_sum<32>(ss);
        raw = group_sum<32>(raw);
        return raw * rms_inv(ss / (float)a->D + 1e-5f);
    }
    return group_sum<32>(dot_chunks<ITD, 32>(R.wD, xr, nD4, sub));
}

// The classifier's two halves of dot_d: its rows all take the same
// RMSNorm'd input, so the lane's columns of it are computed once (the same
// operations as dot_d's, so the sums are bit-identical), and each row block
// is a dot of those against the block's weights.
template <int ITD, int ITH, int GA>
__device__ __forceinline__ void norm_x_d(const PTMI_CONST StepArgs *a, const Regs<ITD, ITH, GA> &R, const float *xs,
                                         float4 (&xr)[ITD]) {
    const int nD4 = a->D >> 2, sub = sub_d();
    read_xs<ITD, 32>(xs, nD4, sub, xr);
    float ss = 0.0f;
#pragma unroll
    for (int it = 0; it < ITD; it++)
        ss = dot4(xr[it], xr[it], ss);
    ss = group_sum<32>(ss);
    const float inv = rms_inv(ss / (float)a->D + 1e-5f);
#pragma unroll
    for (int it = 0; it < ITD; it++) {
        xr[it].x = xr[it].x * inv * R.nw[it].x;
        xr[it].y = xr[it].y * inv * R.nw[it].y;
        xr[it].z = xr[it].z * inv * R.nw[it].z;
        xr[it].w = xr[it].w * inv * R.nw[it].w;
    }
}
template <int ITD>
__device__ __forceinline__ void load_rows_d(const PTMI_CONST StepArgs *a, float4 (&w)[ITD], const float *W, int rows, int rb) {
    const int nD4 = a->D >> 2, sub = sub_d();
    const float *row = W + (long)min(rb * kRowsD + slot_d(), rows - 1) * a->D;
#pragma unroll
    for (int it = 0; it < ITD; it++) w[it] = ntload4(row + 4 * min(sub + it * 32, nD4 - 1));
}
template <int ITD>
__device__ __forceinline__ float dot_rows_d(const PTMI_CONST StepArgs *a, const float4 (&w)[ITD], const float4 (&xr)[ITD]) {
    const int nD4 = a->D >> 2, sub = sub_d();
    const float acc = dot_chunks<ITD, 32>(w, xr, nD4, sub);
    return group_sum<32>(acc);
}

template <int ITD, int ITH, int GA>
__device__ __forceinline__ float dot_h(const PTMI_CONST StepArgs *a, const Regs<ITD, ITH, GA> &R, const float *xs) {
    const int nH4 = a->H >> 2, sub = opaque((int)threadIdx.x & 63);
    float4 xr[ITH];
    read_xs<ITH, 64>(xs, nH4, sub, xr);
    return group_sum<64>(dot_chunks<ITH, 64>(R.wH, xr, nH4, sub));
}

// K/V rows of attention unit u (head u % NH, chunk u / NH) at positions
// below pos (written by earlier tokens' kernels), clamped into the chunk.
template <int ITD, int ITH, int GA, bool V>
__device__ __forceinline__ void load_kv(const PTMI_CONST StepArgs *a, Regs<ITD, ITH, GA> &R, const Tok &t, int l, int u) {
    using Rg = Regs<ITD, ITH, GA>;
    const int lane = (int)threadIdx.x & 63, wave = opaque((int)threadIdx.x >> 6);
    const int h = u % a->NH, c = u / a->NH;
    const int t0 = c * a->chunk, t_end = min(t0 + a->chunk, t.pos + 1);
    const int slot = opaque(lane / GA), sub = opaque(lane % GA);
    const int sub_c = min(sub, (a->hd >> 2) - 1);
    const long base = (long)l * a->S * a->KV + (long)(h / a->kv_mul) * a->hd + 4 * sub_c;
    const int top = max(t0, min(t_end, t.pos) - 1);
#pragma unroll
    for (int q = 0; q < Rg::kU; q++) {
        const int row = t0 + q * (kW * Rg::kRPW) + wave * Rg::kRPW + slot;
        const long o = base + (long)max(t0, min(row, top)) * a->KV;
        if constexpr (V) R.vv[q] = ntload4(a->vc + o);
        else R.kk[q] = ntload4(a->kc + o);
    }
}
// The K rows go out a stage ahead; the V rows only once the unit's q, k and
// v are in (they are first used after the softmax): loaded with the K rows,
// they held back that wait, since a wave's loads complete in order.
template <int ITD, int ITH, int GA>
__device__ __forceinline__ void load_k(const PTMI_CONST StepArgs *a, Regs<ITD, ITH, GA> &R, const Tok &t, int l, int u) {
    load_kv<ITD, ITH, GA, false>(a, R, t, l, u);
}
template <int ITD, int ITH, int GA>
__device__ __forceinline__ void load_v(const PTMI_CONST StepArgs *a, Regs<ITD, ITH, GA> &R, const Tok &t, int l, int u) {
    load_kv<ITD, ITH, GA, true>(a, R, t, l, u);
}

// L2 prefetch by a workgroup that has no work in the current window: row
// blocks rb (rows [rb*R, rb*R + R) of W, n floats per row) that workgroups
// on this XCD (rb % 8 == blockIdx.x % 8) will load into registers later,
// shared among the idle workgroups of this XCD whose blockIdx is at least
// first_idle.  Plain loads allocate the lines in this XCD's L2, which no
// kernel boundary invalidates before the owners read them.
__device__ __forceinline__ float prefetch_rows(const float *W, int rows, int n, int R, int nblocks, int first_idle,
                                               int nb, float acc) {
    const int b = blockIdx.x, x = b & 7;
    if (b < first_idle) return acc;
    const int m0 = first_idle > x ? (first_idle - x + 7) / 8 : 0;
    const int m_end = (nb - 1 - x) / 8 + 1;
    const int rank = b / 8 - m0, nranks = m_end - m0;
    if (nranks <= 0) return acc;
    const int t = opaque((int)threadIdx.x);
    for (int j = rank; x + 8 * j < nblocks; j += nranks) {
        const int rb = x + 8 * j;
        const int r0 = rb * R, r1 = min(r0 + R, rows);
        const long n4 = (long)(r1 - r0) * n / 4;
        const float *base = W + (long)r0 * n;
        for (long i = t; i < n4; i += 8L * kT) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = load4(base + 4 * min(i + (long)u * kT, n4 - 1));
#pragma unroll
            for (int u = 0; u < 8; u++) acc += v[u].x;
        }
    }
    return acc;
}

// Row block rb (R rows of n floats) read into this XCD's L2 by the whole
// workgroup; the values go into acc, which the kernel keeps.
__device__ __forceinline__ float prefetch_block(const float *W, int rows, int n, int R, int rb, float acc) {
    const int r0 = rb * R, r1 = min(r0 + R, rows);
    if (r0 >= r1) return acc;
    const long n4 = (long)(r1 - r0) * n / 4;
    const float *base = W + (long)r0 * n;
    const int t = opaque((int)threadIdx.x);
    for (long i = t; i < n4; i += 8L * kT) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = load4(base + 4 * min(i + (long)u * kT, n4 - 1));
#pragma unroll
        for (int u = 0; u < 8; u++) acc += v[u].x;
    }
    return acc;
}

// Stage g = kStages * layer + s (s: QKV, ATT, WO, W13, W2); g = kStages * L
// is the classifier with the final argmax.  One launch runs stages
// [g0, g1) of the token: the whole step, or a window of it (the host
// splits the step at chosen stages).  Values cross windows through the
// same tagged words; a window loads its first stage's weights at start.
constexpr int kStages = 5;

template <int ITD, int ITH, int GA>
__global__ __launch_bounds__(kT) void k_decode_step(const StepArgs *ap, int g0, int g1) {
    using Rg = Regs<ITD, ITH, GA>;
    // w2's waves store their own rows on the dim-768 instantiation, and
    // hand them to the writer wave on the smaller ones.  Same-box tok/s,
    // writer wave / own stores (w1|w3 storing its own in both): stories110M
    // 6009 / 6075, stories42M 9392 / 8802, stories15M 13043 / 12589.  (A
    // run-time switch between the two cost 0.5-1.2% on every shape.)
    constexpr bool kW2Direct = w2_direct(ITD);
    // Copies of each layer's output x_b (the next QKV input, the last one
    // the classifier's), stored one per wave after the w2 barrier and polled
    // as copy b % kW, where w2 goes through that barrier (the smaller
    // instantiations); with w2's direct stores a single copy.  Same box,
    // tok/s: stories42M 9704-9713 against 9554-9563, stories15M
    // 13257-13324 against 13200-13245; stories110M with the barrier and
    // copies 6139-6141 against 6151-6166 with its direct stores.
    constexpr int kRepXb = rep_xb(ITD);
    // word pairs per polling thread of a dim-length and a hidden-length vector
    constexpr int kPD = (ITD * 64 + kPollT - 1) / kPollT, kPH8 = (ITH * 128 + kT - 1) / kT;
    __shared__ Smem sm;
    Rg R;
    float pf_acc = 0.0f;                              // keeps prefetch loads alive
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.x, nb = gridDim.x;
    auto in = [&](int g) { return g >= g0 && g < g1; };
    Tok tk;
    int L;
    {
        const PTMI_CONST StepArgs *a = fresh(ap);
        // a step or launch window before this one in the same submission
        // failed: its words carry the tag this step would use, so do nothing
        // (the host reports the failure and moves the sequence number on)
        const PTMI_GLOBAL DecodeCtl *ctl = gl(a->ctl);
        const int err = ctl->err;
        tk.pos = ctl->pos;
        tk.tag = (uint32_t)ctl->seq + 1u;
        tk.token = ctl->tok_in;
        if (err) return;
        if (a->stamps && wave == kWriter)
            for (int i = lane; i < a->n_stamps; i += 64) sm.st[i] = 0;
        tk.nact = tk.pos / a->chunk + 1;
        L = a->L;
        if (tid == 0) sm.fail = 0;
        // (a test's check that no chunk merge reads a record it did not poll)
        if (a->poison)
            for (int i = tid; i < kPartLds; i += kT) sm.part[i] = __int_as_float(0x7fc00000);
        // RoPE angle of pair (i, i+1) depends on i % head_dim and pos only
        // (pt_ops.c:33-40): one table per token serves q and k of every layer
        if (tid < (a->hd >> 1)) {
            float c, sn;
            d_rope_cs(2 * tid, a->hd, tk.pos, &c, &sn);
            sm.rope_c[tid] = c;
            sm.rope_s[tid] = sn;
        }
        // the pair of each q/k row of the first QKV block (the same rows in
        // every layer): pair k = (position of the row in its head) / 2
        if (tid >= 64 && tid < 64 + kRowsD) {
            const int r0 = ((b - a->qbase) * kRowsD + tid - 64) & ~1;
            sm.rope_k[tid - 64] = ((r0 < a->D ? r0 : r0 - a->D) % a->hd) >> 1;
        }
        // Each register set is loaded at one point: after the stage that
        // last read it, a stage or more ahead of its use (w1|w3 rows after
        // QKV, w2 rows after Wo, the next QKV or classifier rows after
        // w1|w3, the next K/V and Wo rows after w2).  A load issued from two
        // places would leave the compiler copying registers where the paths
        // join, which waits for the loads there.  A launch loads here what
        // those points before its first stage would have loaded.
        const int D = a->D, H = a->H, QR = D + 2 * a->KV, l = g0 / kStages, k0 = l < L ? g0 % kStages : kStages;
        const int qb = b - a->qbase, wb = b - a->wbase, u = b - a->ubase;
        if (k0 == kStages) {
            if (b < (a->V + kRowsD - 1) / kRowsD) load_wD(a, R, a->wcls, a->V, b, a->rms_final);
        } else {
            if (k0 == 0) {
                if (qb >= 0 && qb < (QR + kRowsD - 1) / kRowsD)
                    load_wD(a, R, a->wqkv + (long)l * QR * D, QR, qb, a->rms_att + (long)l * D);
            } else if (k0 <= 3) {
                if (in(kStages * l + 3) && b < (2 * H + kRowsD - 1) / kRowsD)
                    load_wD(a, R, a->w13 + (long)l * 2 * H * D, 2 * H, b, a->rms_ffn + (long)l * D);
            } else if (in(kStages * (l + 1))) {
                if (l + 1 == L) {
                    if (b < (a->V + kRowsD - 1) / kRowsD) load_wD(a, R, a->wcls, a->V, b, a->rms_final);
                } else if (qb >= 0 && qb < (QR + kRowsD - 1) / kRowsD) {
                    load_wD(a, R, a->wqkv + (long)(l + 1) * QR * D, QR, qb, a->rms_att + (long)(l + 1) * D);
                }
            }
            if (k0 <= 2) {
                // (a window from QKV loads them after its QKV stage)
                if (k0 > 0 && in(kStages * l + 2) && wb >= 0 && wb < (D + kRowsD - 1) / kRowsD) load_wo(a, R, l, wb);
            } else if (in(kStages * l + 4) && b < (D + kRowsH - 1) / kRowsH) {
                load_wH(a, R, a->w2 + (long)l * D * H, D, b);
            }
            if (k0 <= 1 && in(kStages * l + 1) && u >= 0 && u < a->NH * a->n_chunks && u / a->NH < tk.nact)
                load_k(a, R, tk, l, u);
        }
        if (g0 == 0) stamp(a, sm.st, 0);
    }
    __syncthreads();

    for (int l = g0 / kStages; l < L && kStages * l < g1; l++) {
        // ── QKV: y = [Wq;Wk;Wv] . rmsnorm(x), RoPE on q and k (llama2.c:
        //    143-151); k and v also into the cache row of pos ──
        if (in(kStages * l)) {
            const PTMI_CONST StepArgs *a = fresh(ap);
            const int D = a->D, KV = a->KV, QR = D + 2 * KV;
            const int blocks_qkv = (QR + kRowsD - 1) / kRowsD, blocks_wo = (D + kRowsD - 1) / kRowsD;
            const int n_units = a->NH * a->n_chunks;
            const int wb = b - a->wbase;
            const bool pre_wo = in(kStages * l + 2) && wb >= 0 && wb < blocks_wo;
            const int qb = b - a->qbase;
            if (qb >= 0 && qb < blocks_qkv) {
                __syncthreads();                              // xs is free again
                bool ok = true;
                if (l == 0) {
                    const float *x = a->emb + (long)tk.token * D;
                    for (int i = tid; i < D; i += kT) sm.xs[i] = gl(x)[i];
                } else {
                    const uint64_t *src = a->t_xb + (long)(l - 1) * D;
                    if constexpr (kRepXb > 1) src += (long)(b % kRepXb) * a->L * D;
                    ok = tid >= kPollT || poll_pairs<kPD>(src, D, tk.tag, sm.xs, a, tid);
                }
                if (!block_ok(ok, &sm.fail, a->ctl)) return;
                stamp(a, sm.st, 1 + 10 * l);
                // the WO residual rows are rows of this same input
                if (pre_wo && tid < kRowsD) sm.xres[tid] = sm.xs[min(wb * kRowsD + tid, D - 1)];
                uint64_t *t_qkv = a->t_qkv + (long)l * QR;
                for (int rb = qb; rb < blocks_qkv; rb += nb) {
                    if (rb != qb) {
                        __syncthreads();                      // the writer wave is done with yout
                        load_wD(a, R, a->wqkv + (long)l * QR * D, QR, rb, a->rms_att + (long)l * D);
                    }
                    const float acc = dot_d(a, R, sm.xs, true);
                    // RoPE pairs: rows 2k (lanes 0-31) and 2k+1 (lanes 32-63) of a wave
                    const LanePair pr = pl32(acc);
                    const int r = rb * kRowsD + slot_d();
                    if ((lane & 31) == 0 && r < QR) {
                        const int r0 = r & ~1;
                        float out;
                        if (r0 < D + KV) {
                            const int k = rb == qb ? sm.rope_k[slot_d()] : ((r0 < D ? r0 : r0 - D) % a->hd) >> 1;
                            const float c = sm.rope_c[k], sn = sm.rope_s[k];
                            out = (r & 1) ? pr.lo * sn + pr.hi * c : pr.lo * c - pr.hi * sn;
                        } else {
                            out = (r & 1) ? pr.hi : pr.lo;
                        }
                        sm.yout[slot_d()] = out;
                    }
                    __syncthreads();
                    if (wave == kWriter && lane < kRowsD) {
                        const int rw = rb * kRowsD + lane;
                        if (rw < QR) {
                            const float out = sm.yout[lane];
                            // the cache row's address from the two (uniform)
                            // base pointers, so no lane loads a pointer: a
                            // load here would wait for the tagged store above
                            float *const kc = a->kc, *const vc = a->vc;
                            const long crow = ((long)l * a->S + tk.pos) * KV;
                            float *cp = rw >= D + KV ? vc + crow + (rw - D - KV) : kc + crow + (rw - D);
                            tstore(t_qkv + rw, out, tk.tag);
                            if (rw >= D) *gl(cp) = out;
                        }
                    }
                }
                stamp(a, sm.st, 2 + 10 * l);
            } else if (pre_wo) {
                // a Wo block without QKV rows takes its residual rows here
                __syncthreads();
                bool ok = true;
                if (tid < kRowsD) {
                    if (l == 0) sm.xres[tid] = gl(a->emb + (long)tk.token * D)[min(wb * kRowsD + tid, D - 1)];
                    else ok = poll_words<1>(a->t_xb + (long)(l - 1) * D + wb * kRowsD, min(kRowsD, D - wb * kRowsD),
                                            tk.tag, sm.xres, a, tid);
                }
                if (!block_ok(ok, &sm.fail, a->ctl)) return;
            }
            // after QKV: this layer's w1|w3 rows (used in W13) and Wo rows
            // (the Wo blocks sit on QKV workgroups: loaded before the QKV
            // wait, they held it back, since a wave's loads complete in order)
            const int H = a->H;
            if (in(kStages * l + 3) && b < (2 * H + kRowsD - 1) / kRowsD)
                load_wD(a, R, a->w13 + (long)l * 2 * H * D, 2 * H, b, a->rms_ffn + (long)l * D);
            if (pre_wo) load_wo(a, R, l, wb);
            // Workgroups with no QKV, attention or Wo work wait until the
            // w1|w3 stage: meanwhile they stage this layer's w1|w3 and w2
            // rows in their XCD's L2 (and through it the MALL).
            const int first_idle = max(max(a->qbase + blocks_qkv, a->wbase + blocks_wo), a->ubase + n_units);
            if (b >= first_idle && (a->l2pf & 1)) {
                pf_acc = prefetch_rows(a->w13 + (long)l * 2 * H * D, 2 * H, D, kRowsD, (2 * H + kRowsD - 1) / kRowsD,
                                       first_idle, nb, pf_acc);
                pf_acc = prefetch_rows(a->w2 + (long)l * D * H, D, H, kRowsH, (D + kRowsH - 1) / kRowsH, first_idle, nb,
                                       pf_acc);
            }
        }

        // ── ATT: unit (head h, chunk c) over positions [t0, t_end) (llama2.c:
        //    153-177): scores, the chunk's softmax statistics and e.v ──
        if (in(kStages * l + 1)) {
            const PTMI_CONST StepArgs *a = fresh(ap);
            const int D = a->D, KV = a->KV, hd = a->hd, NH = a->NH, QR = D + 2 * KV;
            // one unit per workgroup: the plan keeps every unit on a
            // workgroup of its own (ubase + units <= workgroups), so no unit
            // ever waits behind another unit of the same workgroup
            const int u = b - a->ubase;
            if (u >= 0 && u < NH * a->n_chunks && u / NH < tk.nact) {
                const int h = u % NH, c = u / NH;
                const int t0 = c * a->chunk, t_end = min(t0 + a->chunk, tk.pos + 1), cnt = t_end - t0;
                const bool has_pos = tk.pos < t_end;
                const int kvh = h / a->kv_mul;
                const uint64_t *t_qkv = a->t_qkv + (long)l * QR;
                __syncthreads();
                bool ok = true;
                if (tid < hd) {
                    ok = poll_words<1>(t_qkv + h * hd, hd, tk.tag, sm.qs, a, tid);
                } else if (has_pos && tid >= 128 && tid < 128 + hd) {
                    ok = poll_words<1>(t_qkv + D + kvh * hd, hd, tk.tag, sm.kp, a, tid - 128);
                } else if (has_pos && tid >= 256 && tid < 256 + hd) {
                    ok = poll_words<1>(t_qkv + D + KV + kvh * hd, hd, tk.tag, sm.vp, a, tid - 256);
                }
                if (!block_ok(ok, &sm.fail, a->ctl)) return;
                stamp(a, sm.st, 3 + 10 * l);
                // the V rows, first used after the softmax: issued once q, k
                // and v are in (loaded with the K rows a stage ahead, they
                // held back that wait, since a wave's loads complete in order)
                load_v(a, R, tk, l, u);
                // Every row pass of the unit at once, so the passes'
                // dependency chains (dots, cross-lane sums) overlap instead
                // of running one after another; rows past the unit's
                // positions are computed and dropped.  Row pos is this
                // token's: its key and value come from the polled k and v.
                const float scale = a->att_scale;
                const int slot = lane / GA, sub = lane % GA;
                const bool has = sub < (hd >> 2);
                const int sub_c = has ? sub : 0;
                const float4 q4 = sel4(has, reinterpret_cast<const float4 *>(sm.qs)[sub_c]);
                const float4 kp4 = reinterpret_cast<const float4 *>(sm.kp)[sub_c];
                float spos = dot4(kp4, q4, 0.0f);             // q . k of row pos
                float sv[Rg::kU];
#pragma unroll
                for (int q = 0; q < Rg::kU; q++) sv[q] = dot4(R.kk[q], q4, 0.0f);
                // the row sums over each group of GA lanes, the passes interleaved
                static_assert(GA == 16, "row sums over rows of 16 lanes");
                spos = group_sum<GA>(spos);
#pragma unroll
                for (int q = 0; q < Rg::kU; q++) sv[q] += dpp_xor1(sv[q]);
#pragma unroll
                for (int q = 0; q < Rg::kU; q++) sv[q] += dpp_xor2(sv[q]);
#pragma unroll
                for (int q = 0; q < Rg::kU; q++) sv[q] += dpp_hmirror(sv[q]);
#pragma unroll
                for (int q = 0; q < Rg::kU; q++) sv[q] += dpp_mirror(sv[q]);
                // scaled scores to LDS (one lane per row) and the wave's maximum
                float mx = -INFINITY;
#pragma unroll
                for (int q = 0; q < Rg::kU; q++) {
                    const int t = t0 + q * (kW * Rg::kRPW) + wave * Rg::kRPW + slot;
                    const float scv = (t == tk.pos ? spos : sv[q]) * scale;
                    if (t < t_end) {
                        mx = fmaxf(mx, scv);
                        if (sub == 0) sm.sc[t - t0] = scv;
                    }
                }
                {
                    const LanePair p16 = pl16(mx);
                    mx = fmaxf(p16.lo, p16.hi);
                    const LanePair p32 = pl32(mx);
                    mx = fmaxf(p32.lo, p32.hi);
                }
                if (lane == 0) sm.wred[wave] = mx;
                __syncthreads();
                // chunk softmax statistics: the maximum, then e^(s - max)
                // (one per thread) and their sum
                mx = sm.wred[0];
#pragma unroll
                for (int w = 1; w < kW; w++) mx = fmaxf(mx, sm.wred[w]);
                float sum = 0.0f;
                if (tid < cnt) {
                    const float e = d_expf(sm.sc[tid] - mx);
                    sm.sc[tid] = e;
                    sum = e;
                }
                sum = group_sum<64>(sum);
                if (lane == 0) sm.wred2[wave] = sum;
                __syncthreads();
                // e . v over the unit's rows, every pass's weight read before use
                float ew[Rg::kU];
#pragma unroll
                for (int q = 0; q < Rg::kU; q++)
                    ew[q] = sm.sc[min(q * (kW * Rg::kRPW) + wave * Rg::kRPW + slot, kAttRows - 1)];
                const float4 vp4 = reinterpret_cast<const float4 *>(sm.vp)[sub_c];
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int q = 0; q < Rg::kU; q++) {
                    const int t = t0 + q * (kW * Rg::kRPW) + wave * Rg::kRPW + slot;
                    const float e = t < t_end ? ew[q] : 0.0f;
                    const float4 v4 = sel4(t < t_end, t == tk.pos ? vp4 : R.vv[q]);
                    acc.x = fmaf(e, v4.x, acc.x);
                    acc.y = fmaf(e, v4.y, acc.y);
                    acc.z = fmaf(e, v4.z, acc.z);
                    acc.w = fmaf(e, v4.w, acc.w);
                }
                // sum over the wave's row slots (lanes with equal lane % GA)
                acc.x = xsum32(xsum16(acc.x));
                acc.y = xsum32(xsum16(acc.y));
                acc.z = xsum32(xsum16(acc.z));
                acc.w = xsum32(xsum16(acc.w));
                if (slot == 0 && has) {
                    sm.red[wave][4 * sub + 0] = acc.x;
                    sm.red[wave][4 * sub + 1] = acc.y;
                    sm.red[wave][4 * sub + 2] = acc.z;
                    sm.red[wave][4 * sub + 3] = acc.w;
                }
                __syncthreads();
                // the chunk's record: o = sum_t e_t v_t, max, sum_t e_t
                auto rec_o = [&](int d) {
                    float o = 0.0f;
#pragma unroll
                    for (int w = 0; w < kW; w++) o += sm.red[w][d];
                    return o;
                };
                auto rec_l = [&]() {
                    float ls = 0.0f;
#pragma unroll
                    for (int w = 0; w < kW; w++) ls += sm.wred2[w];
                    return ls;
                };
                uint64_t *head_part = a->t_part + ((long)l * NH + h) * a->n_chunks * (hd + 2);
                if (c > 0) {
                    // a later chunk: its record (o, max, sum) goes to the
                    // head's chunk-0 unit
                    uint64_t *dst = head_part + (long)c * (hd + 2);
                    if (wave == kWriter) {
                        // the record's LDS reads all before its first store:
                        // a read into registers that a store still holds
                        // would wait for that store's acknowledgement
                        float o = rec_o(min(lane, hd - 1)), ls = rec_l();
                        asm volatile("" : "+v"(o), "+v"(ls));
                        if (lane < hd) tstore(dst + lane, o, tk.tag);
                        if (lane == 0) tstore(dst + hd, mx, tk.tag);
                        if (lane == 1) tstore(dst + hd + 1, ls, tk.tag);
                    }
                } else {
                    // chunk 0 merges the head's active chunks: its own
                    // record (put in LDS slot 0 by the writer wave) and the
                    // others' (polled into slots 1..), then w_c =
                    // e^(m_c - M) / sum_c' l_c' e^(m_c' - M) and out =
                    // sum_c w_c o_c, published for the WO stage.  One chunk
                    // is o / l, which is what the general arithmetic gives
                    // there (M = m, e^0 = 1); the writer wave stores it
                    // directly.  With several, all eight waves merge (the
                    // writer wave alone took 0.84-0.90 us at long context,
                    // a chain of per-chunk LDS reads and broadcasts).
                    static_assert(kMaxChunks == 8, "chunk statistics reduce over 8-lane groups");
                    const int nact = tk.nact, nother = nact - 1;
                    float o0 = 0.0f, l0 = 0.0f;
                    if (wave == kWriter) {
                        o0 = rec_o(min(lane, hd - 1));
                        l0 = rec_l();
                        if (nact > 1) {
                            // its own record into slot 0, beside the polled ones
                            if (lane < hd) sm.part[lane] = o0;
                            if (lane == 0) sm.part[hd] = mx;
                            if (lane == 1) sm.part[hd + 1] = l0;
                        }
                    }
                    bool ok = true;
                    if (nother > 0 && tid < kPollT)
                        ok = poll_pairs<1>(head_part + (hd + 2), nother * (hd + 2), tk.tag, sm.part + (hd + 2), a, tid);
                    if (!block_ok(ok, &sm.fail, a->ctl)) return;
                    if (nact == 1) {
                        if (wave == kWriter && lane < hd)
                            tstore(a->t_att + (long)l * D + h * hd + lane, o0 * (1.0f / l0), tk.tag);
                    } else {
                        // every wave merges 8 of the head's outputs: lane 8g + k
                        // takes output wave*8 + g of chunk k; the chunk
                        // statistics and the weighted sum reduce over the
                        // lane's 8-lane group (three cross-lane steps each)
                        const int k = lane & 7, dq = wave * 8 + (lane >> 3), dd = min(dq, hd - 1);
                        const bool act = k < nact;
                        const float *pc = sm.part + k * (hd + 2);
                        const float mc = pc[hd], lc = pc[hd + 1], oc = pc[dd];
                        // (inactive chunks' LDS records were not written this
                        // token: their values, possibly not finite, are
                        // selected out, never multiplied by zero)
                        float M = act ? mc : -INFINITY;
                        M = fmaxf(M, dpp_xor1(M));
                        M = fmaxf(M, dpp_xor2(M));
                        M = fmaxf(M, dpp_hmirror(M));
                        const float f = act ? d_expf(mc - M) : 0.0f;
                        float Ls = act ? lc * f : 0.0f;
                        Ls += dpp_xor1(Ls);
                        Ls += dpp_xor2(Ls);
                        Ls += dpp_hmirror(Ls);
                        float pv = act ? oc * (f * (1.0f / Ls)) : 0.0f;
                        pv += dpp_xor1(pv);
                        pv += dpp_xor2(pv);
                        pv += dpp_hmirror(pv);
                        if (k == 0 && dq < hd) sm.mrg[dq] = pv;
                        __syncthreads();
                        if (wave == kWriter && lane < hd) tstore(a->t_att + (long)l * D + h * hd + lane, sm.mrg[lane], tk.tag);
                    }
                }
                stamp(a, sm.st, 4 + 10 * l);
            }
        }

        // ── WO: x_a = x + Wo . att (llama2.c:179-180) ──
        if (in(kStages * l + 2)) {
            const PTMI_CONST StepArgs *a = fresh(ap);
            const int D = a->D, H = a->H;
            const int blocks_wo = (D + kRowsD - 1) / kRowsD;
            const float *x_emb = a->emb + (long)tk.token * D;
            const uint64_t *t_xin = a->t_xb + (long)(l - 1) * D;      // used for l > 0 only
            uint64_t *t_xa = a->t_xa + (long)l * D;
            const int wb = b - a->wbase;
            if (wb >= 0 && wb < blocks_wo) {
                __syncthreads();
                bool ok = tid >= kPollT || poll_pairs<kPD>(a->t_att + (long)l * D, D, tk.tag, sm.xs, a, tid);
                if (!block_ok(ok, &sm.fail, a->ctl)) return;
                stamp(a, sm.st, 5 + 10 * l);
                // the residual rows came with this layer's QKV input when the
                // QKV stage ran in this launch; otherwise they are read here
                const bool res_here = !in(kStages * l);
                for (int rb = wb; rb < blocks_wo; rb += nb) {
                    if (rb != wb || res_here) {
                        __syncthreads();                      // the writer wave is done with yout
                        if (rb != wb) load_wo(a, R, l, rb);
                        bool ok2 = true;
                        if (tid < kRowsD) {
                            if (l == 0) sm.xres[tid] = gl(x_emb)[min(rb * kRowsD + tid, D - 1)];
                            else ok2 = poll_words<1>(t_xin + rb * kRowsD, min(kRowsD, D - rb * kRowsD), tk.tag, sm.xres, a, tid);
                        }
                        if (!block_ok(ok2, &sm.fail, a->ctl)) return;
                    }
                    const float acc = dot_wo(a, R, sm.xs);
                    const int slot = slot_d();
                    if ((lane & 31) == 0) sm.yout[slot] = sm.xres[slot] + acc;
                    __syncthreads();
                    if (wave == kWriter && lane < kRowsD && rb * kRowsD + lane < D) {
#pragma unroll
                        for (int r = 0; r < kRepXa; r++)
                            tstore(t_xa + (long)r * a->L * D + rb * kRowsD + lane, sm.yout[lane], tk.tag);
                    }
                }
                stamp(a, sm.st, 6 + 10 * l);
            }
            // after Wo: this layer's w2 rows (used in W2)
            if (in(kStages * l + 4) && b < (D + kRowsH - 1) / kRowsH) load_wH(a, R, a->w2 + (long)l * D * H, D, b);
        }

        // ── W13: hb = silu(w1 . xn) * (w3 . xn), xn = rmsnorm(x_a)
        //    (llama2.c:184-188; w1/w3 rows interleaved) ──
        if (in(kStages * l + 3)) {
            const PTMI_CONST StepArgs *a = fresh(ap);
            const int D = a->D, H = a->H;
            const int blocks_w13 = (2 * H + kRowsD - 1) / kRowsD, blocks_w2 = (D + kRowsH - 1) / kRowsH;
            if (b < blocks_w13) {
                __syncthreads();                              // xs and xres2 are free again
                bool ok = tid >= kPollT ||
                          poll_pairs<kPD>(a->t_xa + (long)(b % kRepXa) * a->L * D + (long)l * D, D, tk.tag, sm.xs, a, tid);
                if (!block_ok(ok, &sm.fail, a->ctl)) return;
                stamp(a, sm.st, 7 + 10 * l);
                // the W2 residual rows are rows of this same input
                if (b < blocks_w2 && tid < kRowsH) sm.xres2[tid] = sm.xs[min(b * kRowsH + tid, D - 1)];
                uint64_t *t_hb = a->t_hb + (long)l * H;
                for (int rb = b; rb < blocks_w13; rb += nb) {
                    if (rb != b) {
                        __syncthreads();                      // every wave is done with the block before
                        load_wD(a, R, a->w13 + (long)l * 2 * H * D, 2 * H, rb, a->rms_ffn + (long)l * D);
                    }
                    const float acc = dot_d(a, R, sm.xs, true);
                    const LanePair pr = pl32(acc);
                    // Each wave stores its own output (no barrier, no writer
                    // wave): the waves' next poll (w2's, right after) may wait
                    // for the acknowledgement of these stores, but it cannot
                    // complete before the last w1|w3 workgroup's words land
                    // anyway (stories110M 6009 against 5949 tok/s, 6075 with
                    // w2 storing its own too; stories42M 9392 against 9373;
                    // same box).  Storing Wo's outputs this way delayed the
                    // w1|w3 release by 1.5 us (Wo's 16 words per block from
                    // 16 single-lane stores, polled by every workgroup), the
                    // merged head outputs likewise Wo's release by 0.25 us,
                    // and QKV's added the cache-row work to the storing
                    // lanes; those keep the writer wave.
                    const int i = rb * (kRowsD / 2) + wave;       // hb index of this wave's row pair
                    if (lane == 0 && 2 * i < 2 * H) {
                        const float h1 = pr.lo, h3 = pr.hi;
                        const float sg = h1 / (1.0f + d_expf(-h1));
                        tstore(t_hb + i, sg * h3, tk.tag);
                    }
                }
                stamp(a, sm.st, 8 + 10 * l);
            }
            // after W13: the next layer's QKV rows, or the classifier's
            if (in(kStages * (l + 1))) {
                const int QR = D + 2 * a->KV, qb = b - a->qbase;
                if (l + 1 == a->L) {
                    if (b < (a->V + kRowsD - 1) / kRowsD) load_wD(a, R, a->wcls, a->V, b, a->rms_final);
                } else if (qb >= 0 && qb < (QR + kRowsD - 1) / kRowsD) {
                    load_wD(a, R, a->wqkv + (long)(l + 1) * QR * D, QR, qb, a->rms_att + (long)(l + 1) * D);
                }
            }
        }

        // ── W2: x_b = x_a + w2 . hb (llama2.c:189-190) ──
        if (in(kStages * l + 4)) {
            const PTMI_CONST StepArgs *a = fresh(ap);
            const int D = a->D, H = a->H, QR = D + 2 * a->KV;
            const int blocks_w2 = (D + kRowsH - 1) / kRowsH, blocks_w13 = (2 * H + kRowsD - 1) / kRowsD;
            const bool last_layer = l + 1 == a->L;
            if (b < blocks_w2) {
                const uint64_t *t_xa = a->t_xa + (long)l * D;
                uint64_t *t_xb = a->t_xb + (long)l * D;
                __syncthreads();
                // every wave polls the hidden vector, the writer wave too
                // (its hb stores of the stage before are acknowledged about
                // as soon as the other waves' first round is back)
                bool ok = poll_pairs<kPH8, kT>(a->t_hb + (long)l * H, H, tk.tag, sm.xs, a, tid);
                if (ok && tid < kRowsH && (b >= blocks_w13 || !in(kStages * l + 3)))   // residual rows not taken in W13
                    ok = poll_words<1>(t_xa + b * kRowsH, min(kRowsH, D - b * kRowsH), tk.tag, sm.xres2, a, tid);
                if (!block_ok(ok, &sm.fail, a->ctl)) return;
                stamp(a, sm.st, 9 + 10 * l);
                for (int rb = b; rb < blocks_w2; rb += nb) {
                    if (rb != b) {
                        __syncthreads();                      // every wave is done with the block before
                        load_wH(a, R, a->w2 + (long)l * D * H, D, rb);
                        bool ok2 = true;
                        if (tid < kRowsH)
                            ok2 = poll_words<1>(t_xa + rb * kRowsH, min(kRowsH, D - rb * kRowsH), tk.tag, sm.xres2, a, tid);
                        if (!block_ok(ok2, &sm.fail, a->ctl)) return;
                    }
                    const float acc = dot_h(a, R, sm.xs);
                    if constexpr (kW2Direct) {                // each wave stores its own row
                        if (lane == 0 && rb * kRowsH + wave < D)
                            tstore(t_xb + rb * kRowsH + wave, sm.xres2[wave] + acc, tk.tag);
                    } else {
                        if (lane == 0) sm.yout[wave] = sm.xres2[wave] + acc;
                        __syncthreads();
                        // wave r stores copy r of the block's kRowsH values
                        if (lane < kRowsH && rb * kRowsH + lane < D)
                            tstore(t_xb + (long)wave * a->L * D + rb * kRowsH + lane, sm.yout[lane], tk.tag);
                    }
                }
                stamp(a, sm.st, 10 + 10 * l);
            } else {
                // idle until the next layer's QKV input: stage its QKV and Wo
                // rows in this XCD's L2
                if (!last_layer && (a->l2pf & 2)) {
                    // (with the QKV blocks past the w2 blocks, their rows are
                    // already in registers, and so are the Wo rows of the Wo
                    // blocks on QKV workgroups)
                    if (a->qbase == 0)
                        pf_acc = prefetch_rows(a->wqkv + (long)(l + 1) * QR * D, QR, D, kRowsD, (QR + kRowsD - 1) / kRowsD,
                                               blocks_w2, nb, pf_acc);
                    if (a->wbase == 0)
                        pf_acc = prefetch_rows(a->wo + (long)(l + 1) * D * D, D, D, kRowsD, (D + kRowsD - 1) / kRowsD,
                                               blocks_w2, nb, pf_acc);
                } else if (last_layer && in(kStages * L)) {
                    // the last layer: this workgroup's classifier row blocks
                    // after the two the classifier starts with
                    for (int j = 0; j < a->cls_pf; j++)
                        pf_acc = prefetch_block(a->wcls, a->V, D, kRowsD, b + (2 + j) * nb, pf_acc);
                }
            }
            // after W2: the next layer's K/V rows (attention units)
            if (!last_layer) {
                const int u = b - a->ubase;
                if (in(kStages * (l + 1) + 1) && u >= 0 && u < a->NH * a->n_chunks && u / a->NH < tk.nact)
                    load_k(a, R, tk, l + 1, u);
            }
        }
    }
    if (pf_acc == 1.2345e-37f) sm.fail = 2;            // never true: keeps the prefetch loads
    if (!in(kStages * L)) {                           // the classifier is in a later launch
        flush_stamps(fresh(ap), sm.st);
        return;
    }

    // ── classifier: logits = Wcls . rmsnorm(x) (llama2.c:195-197), and this
    //    workgroup's argmax candidate ──
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    {
        const PTMI_CONST StepArgs *a = fresh(ap);
        const int blocks_cls = (a->V + kRowsD - 1) / kRowsD;
        if (b < blocks_cls) {
            // Two row blocks in flight: R.wD holds block b (loaded during the
            // last layer), wB the next one, issued before the wait for x.
            // Each block's loads go out as soon as the block two before it
            // is consumed.
            float4 wB[ITD], xr[ITD];
            if (b + nb < blocks_cls) load_rows_d(a, wB, a->wcls, a->V, b + nb);
            __syncthreads();
            const uint64_t *src = a->t_xb + (long)(a->L - 1) * a->D;
            if constexpr (kRepXb > 1) src += (long)(b % kRepXb) * a->L * a->D;
            bool ok = tid >= kPollT || poll_pairs<kPD>(src, a->D, tk.tag, sm.xs, a, tid);
            if (!block_ok(ok, &sm.fail, a->ctl)) return;
            stamp(a, sm.st, 1 + 10 * a->L);
            norm_x_d(a, R, sm.xs, xr);
            // one row block: its logits (ycls[p], stored by the writer wave)
            // and this lane's argmax candidate.  ycls alternates, so the
            // barrier of the next block also orders the writer's reads of
            // this one before the block after overwrites it.
            auto block = [&](const float4 (&w)[ITD], int rb, int p) {
                const float acc = dot_rows_d(a, w, xr);
                const int r = rb * kRowsD + slot_d();
                if (r < a->V) {
                    if ((lane & 31) == 0) sm.ycls[p][slot_d()] = acc;
                    take_best(bv, bi, acc, r);
                }
            };
            auto store = [&](int rb, int p) {
                __syncthreads();
                if (wave == kWriter && lane < kRowsD && rb * kRowsD + lane < a->V)
                    gl(a->logits)[rb * kRowsD + lane] = sm.ycls[p][lane];
            };
            for (int rb = b; rb < blocks_cls; rb += 2 * nb) {
                block(R.wD, rb, 0);
                if (rb + 2 * nb < blocks_cls) load_rows_d(a, R.wD, a->wcls, a->V, rb + 2 * nb);
                store(rb, 0);
                if (rb + nb >= blocks_cls) break;
                block(wB, rb + nb, 1);
                if (rb + 3 * nb < blocks_cls) load_rows_d(a, wB, a->wcls, a->V, rb + 3 * nb);
                store(rb + nb, 1);
            }
            stamp(a, sm.st, 2 + 10 * a->L);
        }
    }
    // workgroup argmax: DPP within rows of 16, the permlane swaps, then
    // across waves
    auto dpp_pair = [&](auto ctrl) {
        constexpr int C = decltype(ctrl)::value;
        take_best(bv, bi, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(bv), C, 0xF, 0xF, true)),
                  __builtin_amdgcn_mov_dpp(bi, C, 0xF, 0xF, true));
    };
    dpp_pair(std::integral_constant<int, 0xB1>{});
    dpp_pair(std::integral_constant<int, 0x4E>{});
    dpp_pair(std::integral_constant<int, 0x141>{});
    dpp_pair(std::integral_constant<int, 0x140>{});
    {
        int ih;
        const int il = pl16i(bi, ih);
        const LanePair p = pl16(bv);
        bv = p.lo; bi = il;
        take_best(bv, bi, p.hi, ih);
    }
    {
        int ih;
        const int il = pl32i(bi, ih);
        const LanePair p = pl32(bv);
        bv = p.lo; bi = il;
        take_best(bv, bi, p.hi, ih);
    }
    __syncthreads();
    if (lane == 0) { sm.ybuf[wave][0] = bv; sm.ybuf[wave][1] = __int_as_float(bi); }
    __syncthreads();
    const PTMI_CONST StepArgs *a = fresh(ap);
    if (tid == kPollT) {                              // the writer wave
        float v = sm.ybuf[0][0];
        int i = __float_as_int(sm.ybuf[0][1]);
        for (int w = 1; w < kW; w++) take_best(v, i, sm.ybuf[w][0], __float_as_int(sm.ybuf[w][1]));
        tstore(a->t_cand + 2 * b, v, tk.tag);
        tstore(a->t_cand + 2 * b + 1, __int_as_float(i), tk.tag);
    }
    if (b != 0) {
        flush_stamps(a, sm.st);
        return;
    }

    // ── workgroup 0: the step's argmax, prompt forcing and position
    //    advance (pt.c:267-271, pt_text.c:344-350) ──
    __syncthreads();
    bool ok = tid >= kPollT || poll_pairs<2>(a->t_cand, 2 * nb, tk.tag, sm.cand, a, tid);
    if (!block_ok(ok, &sm.fail, a->ctl)) return;
    stamp(a, sm.st, 3 + 10 * a->L);
    bv = -INFINITY;
    bi = 0x7fffffff;
    for (int w = tid; w < nb; w += kT) take_best(bv, bi, sm.cand[2 * w], __float_as_int(sm.cand[2 * w + 1]));
    dpp_pair(std::integral_constant<int, 0xB1>{});
    dpp_pair(std::integral_constant<int, 0x4E>{});
    dpp_pair(std::integral_constant<int, 0x141>{});
    dpp_pair(std::integral_constant<int, 0x140>{});
    {
        int ih;
        const int il = pl16i(bi, ih);
        const LanePair p = pl16(bv);
        bv = p.lo; bi = il;
        take_best(bv, bi, p.hi, ih);
    }
    {
        int ih;
        const int il = pl32i(bi, ih);
        const LanePair p = pl32(bv);
        bv = p.lo; bi = il;
        take_best(bv, bi, p.hi, ih);
    }
    __syncthreads();
    if (lane == 0) { sm.ybuf[wave][0] = bv; sm.ybuf[wave][1] = __int_as_float(bi); }
    __syncthreads();
    if (tid == 0) {
        float v = bv;
        int i = bi;
        for (int w = 1; w < kW; w++) take_best(v, i, sm.ybuf[w][0], __float_as_int(sm.ybuf[w][1]));
        // nothing above -inf, or a NaN first logit (pt_ops.c:65-70 keeps
        // index 0 then): 0.  Row 0 is this workgroup's own first row.
        const float l0 = gl(a->logits)[0];
        if (i == 0x7fffffff || l0 != l0) i = 0;
        const int pos = tk.pos;
        PTMI_GLOBAL DecodeCtl *ctl = gl(a->ctl);
        const int next = (pos < ctl->n_prompt - 1) ? gl(a->prompt)[pos + 1] : i;
        ctl->next = i;
        ctl->tok_in = next;
        ctl->pos = pos + 1;
        ctl->seq = (int)tk.tag;
        if (a->out_tokens) gl(a->out_tokens)[pos] = next;
    }
    stamp(a, sm.st, 4 + 10 * a->L);
    flush_stamps(a, sm.st);
}

using StepFn = void (*)(const StepArgs *, int, int);

// Instantiated shapes: (float4 per lane of a D-row, of an H-row, lanes per
// K/V row).  Other shapes keep the multi-kernel step.
struct StepKernel { int itd, ith, ga; StepFn fn; };
const StepKernel kStepKernels[] = {
    {1, 1, 16, k_decode_step<1, 1, 16>}, {2, 2, 16, k_decode_step<2, 2, 16>},
    {3, 3, 16, k_decode_step<3, 3, 16>}, {4, 6, 16, k_decode_step<4, 6, 16>},
    {6, 8, 16, k_decode_step<6, 8, 16>},
};

}  // namespace

// The one-kernel step's launch plan for a model shape, on a device with
// `cus` compute units of which each holds `per_cu` workgroups of the step
// kernel at once (its occupancy).  The step runs one workgroup per compute
// unit, all resident at the same time: the stages hand values to each
// other through memory and wait for them, so a workgroup that has not
// started would make its consumers wait until their bound runs out.  Each
// attention unit needs a workgroup of its own (a head's chunk-0 unit waits
// for the head's other units; queued behind another unit's wait on the
// same workgroup, two merges could wait for each other).  Returns kPlanOk,
// or why the multi-kernel step runs instead.
enum { kPlanOk = 0, kPlanShape = 1, kPlanResident = 2 };
struct StepPlan {
    const StepKernel *k;
    int chunk, n_chunks;   // attention positions per unit, units per head
    int nb, units;         // workgroups, attention units
};
static int plan_step(const Config &c, int cus, int per_cu, StepPlan *p) {
    *p = StepPlan{};
    if (c.dim % 4 || c.hidden % 4 || c.head_dim % 4 || (c.dim & 1) || (c.kv_dim & 1)) return kPlanShape;
    if (c.dim > 2048 || c.hidden > 2048 || c.head_dim > 128 || c.n_heads > 64) return kPlanShape;
    const int itd = (c.dim / 4 + 31) / 32, ith = (c.hidden / 4 + 63) / 64;
    const int ga = 16;                                     // lanes per V row: head_dim <= 64
    if (c.head_dim > 4 * ga || c.n_heads * c.head_dim != c.dim) return kPlanShape;
    // chunk: a multiple of the K/V rows one pass of the workgroup covers,
    // at most kAttRows positions, at most kMaxChunks per head
    const int gran = kW * (64 / ga);
    int ch = (c.seq_len + kMaxChunks - 1) / kMaxChunks;
    ch = (ch + gran - 1) / gran * gran;
    if (ch > kAttRows) return kPlanShape;
    const int nc = (c.seq_len + ch - 1) / ch;
    if (nc * (c.head_dim + 2) > kPartLds) return kPlanShape;
    for (const StepKernel &k : kStepKernels)
        if (k.ga == ga && k.itd >= itd && k.ith >= ith && k.itd <= itd + 1 && k.ith <= ith + 2) {
            p->k = &k;
            break;
        }
    if (!p->k) return kPlanShape;
    p->chunk = ch;
    p->n_chunks = nc;
    p->nb = std::min(cus, 512);
    p->units = c.n_heads * nc;
    if (cus <= 0 || per_cu < 1 || p->units > p->nb) return kPlanResident;
    return kPlanOk;
}

int decode_step_create(ptmi_model *m) {
    // PTMI_DECODE_STEP=1 / 0 forces this step / the captured multi-kernel
    // step.  Unset: this step wherever the plan allows it (measured faster
    // on stories15M, 42M and 110M).
    m->step_plan = -1;
    const char *env = getenv("PTMI_DECODE_STEP");
    const bool on = env && env[0] ? env[0] == '1' : true;
    if (!on) return PTMI_OK;
    StepPlan plan;
    if (plan_step(m->c, 1 << 20, 1, &plan) == kPlanShape) {
        m->step_plan = kPlanShape;
        return PTMI_OK;                                    // multi-kernel step
    }
    int dev = 0, cus = 0, per_cu = 0;
    PTMI_HIP(hipGetDevice(&dev));
    PTMI_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    PTMI_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(plan.k->fn), kT, 0));
    m->step_plan = plan_step(m->c, cus, per_cu, &plan);
    if (m->step_plan != kPlanOk) return PTMI_OK;           // multi-kernel step
    const int chunk = plan.chunk, nc = plan.n_chunks;
    const Config &c = m->c;
    const long L = c.n_layers, D = c.dim, H = c.hidden, KV = c.kv_dim, NH = c.n_heads, hd = c.head_dim;
    const int nb = std::min(cus, 512);
    // tagged words, then the argument block (32-byte aligned)
    const size_t words = L * (D + 2 * KV) + L * nc * NH * (hd + 2) + (1 + kRepXa + rep_xb(plan.k->itd)) * L * D +
                         L * H + 2 * (size_t)nb;
    const char *st_env = getenv("PTMI_STEP_STAMPS");
    const int n_stamps = (st_env && st_env[0] == '1') ? (int)(1 + 10 * L + 4) : 0;
    if (n_stamps > kStampSlots)
        return set_error(PTMI_ERR_ARG, "PTMI_STEP_STAMPS=1: the stamps hold at most 32 layers (model has %ld)", L);
    const size_t args_off = (words * sizeof(uint64_t) + 255) / 256 * 256;
    const size_t stamps_off = (args_off + sizeof(StepArgs) + 255) / 256 * 256;
    const size_t total = stamps_off + (size_t)nb * n_stamps * sizeof(uint64_t);
    char *mem = nullptr;
    PTMI_HIP(hipMalloc(&mem, total));
    const Resident *r = m->res;
    StepArgs a = {};
    a.emb = r->emb; a.rms_att = r->rms_att; a.wqkv = r->wqkv; a.wo = r->wo; a.rms_ffn = r->rms_ffn;
    a.w13 = r->w13; a.w2 = r->w2; a.rms_final = r->rms_final; a.wcls = r->wcls;
    a.D = c.dim; a.H = c.hidden; a.L = c.n_layers; a.NH = c.n_heads; a.KV = c.kv_dim; a.hd = c.head_dim;
    a.kv_mul = c.n_heads / c.n_kv_heads; a.V = c.vocab; a.S = c.seq_len;
    a.chunk = chunk; a.n_chunks = nc;
    // The attention units sit on the workgroups after the QKV row blocks
    // when they fit (PTMI_STEP_UNIT_BASE=0: from workgroup 0), so their K/V
    // loads go out at the start of the QKV stage
    // The QKV row blocks sit on the workgroups after the w2 row blocks (when
    // they fit; PTMI_STEP_QBASE=0: from workgroup 0), which then preload
    // their next-layer QKV rows during w2 (stories15M/42M/110M +2.7/+2.4/
    // +3.4%)
    {
        const char *ub = getenv("PTMI_STEP_UNIT_BASE");
        const char *qs = getenv("PTMI_STEP_QBASE");
        const int blocks_qkv = (int)((D + 2 * KV + kRowsD - 1) / kRowsD), blocks_w2 = (int)((D + kRowsH - 1) / kRowsH);
        a.qbase = (!(qs && qs[0] == '0') && blocks_w2 + blocks_qkv <= nb) ? blocks_w2 : 0;
        // The Wo row blocks sit on the first QKV workgroups (PTMI_STEP_WBASE=0:
        // from workgroup 0), idle between QKV and Wo, so the w2 workgroups
        // are idle in Wo and load their w2 rows then
        const char *ws = getenv("PTMI_STEP_WBASE");
        a.wbase = (ws && ws[0] == '0') ? 0 : a.qbase;
        const bool ub_on = !(ub && ub[0] == '0');
        if (a.qbase > 0)
            a.ubase = NH * nc <= a.qbase ? 0 : (ub_on && a.qbase + blocks_qkv + NH * nc <= nb ? a.qbase + blocks_qkv : 0);
        else
            a.ubase = (ub_on && blocks_qkv + NH * nc <= nb) ? blocks_qkv : 0;
        // (ubase + units <= nb in every case: the plan has units <= nb)
    }
    a.att_scale = host_att_scale(c.head_dim);
    a.kc = m->kc; a.vc = m->vc; a.logits = m->logits; a.ctl = m->ctl;
    a.prompt = m->prompt; a.out_tokens = m->out_tokens;
    uint64_t *p = reinterpret_cast<uint64_t *>(mem);
    a.t_qkv = p;  p += L * (D + 2 * KV);
    a.t_part = p; p += L * nc * NH * (hd + 2);
    a.t_att = p;  p += L * D;
    a.t_xa = p;   p += kRepXa * L * D;
    a.t_xb = p;   p += rep_xb(plan.k->itd) * L * D;
    a.t_hb = p;   p += L * H;
    a.t_cand = p;
    a.stamps = n_stamps ? reinterpret_cast<uint64_t *>(mem + stamps_off) : nullptr;
    a.n_stamps = n_stamps;
    // PTMI_STEP_WAIT_TICKS shortens the bound of every wait (tests of the
    // timeout path: the step then fails and reports, and every wave exits)
    const char *wt = getenv("PTMI_STEP_WAIT_TICKS");
    a.wait_ticks = wt ? strtoull(wt, nullptr, 10) : kWaitTicks;
    // Idle workgroups stage the next stages' weights in L2: this layer's
    // w1|w3 and w2 during QKV (1) only when enough of them are idle (64+:
    // stories15M/42M, +0.2% / +1.7%; with 16 idle on stories110M the staging
    // delays their own w1|w3 rows), the next layer's QKV and Wo during w2 (2)
    // always.  PTMI_STEP_L2PF overrides.
    {
        const int blocks_qkv = (int)((D + 2 * KV + kRowsD - 1) / kRowsD), blocks_wo = (int)((D + kRowsD - 1) / kRowsD);
        const int first_idle = std::max(std::max(a.qbase + blocks_qkv, a.wbase + blocks_wo), a.ubase + (int)(NH * nc));
        const char *pf = getenv("PTMI_STEP_L2PF");
        a.l2pf = pf ? atoi(pf) & 3 : (nb - first_idle >= 64 ? 3 : 2);
        // In the last layer the workgroups idle during w2 also stage the
        // classifier row block they take third (PTMI_STEP_CLSPF: 0-4 blocks)
        const char *cp = getenv("PTMI_STEP_CLSPF");
        a.cls_pf = cp ? std::max(0, std::min(4, atoi(cp))) : 1;
        const char *pz = getenv("PTMI_STEP_POISON_LDS");
        a.poison = pz && pz[0] == '1';
    }
    hipError_t e = hipMemsetAsync(mem, 0, total, lib_stream());
    if (e == hipSuccess) e = hipMemcpyAsync(mem + args_off, &a, sizeof(a), hipMemcpyHostToDevice, lib_stream());
    if (e == hipSuccess) e = hipStreamSynchronize(lib_stream());
    if (e != hipSuccess) { (void)hipFree(mem); return hip_check(e, "set up the decode step"); }
    m->step_mem = reinterpret_cast<uint64_t *>(mem);
    m->step_args = mem + args_off;
    m->step_nb = nb;
    m->step_fn = reinterpret_cast<const void *>(plan.k->fn);
    m->step_chunk = chunk;
    m->step_chunks = nc;
    m->step_stamps = a.stamps;
    m->step_n_stamps = n_stamps;
    // Launch windows: PTMI_STEP_SPLIT names the stages before which a new
    // launch starts, in every layer: q QKV, a attention, o Wo, f w1|w3,
    // d w2, c the classifier.  Unset or empty: one launch per token.
    m->step_cuts.assign(1, 0);
    if (const char *sp = getenv("PTMI_STEP_SPLIT")) {
        static const char kLetters[] = "qaofd";
        for (const char *q = sp; *q; q++)
            if (!strchr("qaofdc", *q)) return set_error(PTMI_ERR_ARG, "PTMI_STEP_SPLIT: unknown stage '%c'", *q);
        for (long g = 1; g <= kStages * L; g++) {
            const bool cut = g == kStages * L ? strchr(sp, 'c') != nullptr : strchr(sp, kLetters[g % kStages]) != nullptr;
            if (cut) m->step_cuts.push_back((int)g);
        }
    }
    m->step_cuts.push_back((int)(kStages * L + 1));
    return PTMI_OK;
}

void decode_step_destroy(ptmi_model *m) {
    if (m->step_mem) (void)hipFree(m->step_mem);
    m->step_mem = nullptr;
    m->step_args = nullptr;
    m->step_fn = nullptr;
}

int decode_step_windows(const ptmi_model *m) { return (int)m->step_cuts.size() - 1; }

int launch_decode_step(ptmi_model *m, int w, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    if (!m->step_fn || !m->step_args) return set_error(PTMI_ERR_STATE, "decode step kernel not set up for this model");
    if (w < 0 || w >= decode_step_windows(m)) return set_error(PTMI_ERR_ARG, "decode step window %d out of range", w);
    const StepArgs *args = reinterpret_cast<const StepArgs *>(m->step_args);
    const StepFn fn = reinterpret_cast<StepFn>(const_cast<void *>(m->step_fn));
    launch_k(fn, dim3(m->step_nb), dim3(kT), 0, s, e0, e1, args, m->step_cuts[w], m->step_cuts[w + 1]);
    PTMI_HIP(hipGetLastError());
    return PTMI_OK;
}

}  // namespace ptmi

using namespace ptmi;

extern "C" int ptmi_decode_step_plan(const int cfg7[7], int cus, int per_cu, int *reason, int *grid, int *units) {
    if (!cfg7 || !reason) return set_error(PTMI_ERR_ARG, "ptmi_decode_step_plan: NULL argument");
    Config c{};
    c.dim = cfg7[0]; c.hidden = cfg7[1]; c.n_layers = cfg7[2]; c.n_heads = cfg7[3]; c.n_kv_heads = cfg7[4];
    c.vocab = cfg7[5]; c.seq_len = cfg7[6];
    if (c.dim <= 0 || c.hidden <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.vocab <= 0 ||
        c.seq_len <= 0 || c.dim % c.n_heads || c.n_heads % c.n_kv_heads)
        return set_error(PTMI_ERR_ARG, "ptmi_decode_step_plan: bad shape");
    c.head_dim = c.dim / c.n_heads;
    c.kv_dim = c.n_kv_heads * c.head_dim;
    StepPlan p;
    *reason = plan_step(c, cus, per_cu, &p);
    if (grid) *grid = *reason == kPlanShape ? 0 : p.nb;
    if (units) *units = *reason == kPlanShape ? 0 : p.units;
    return PTMI_OK;
}

extern "C" int ptmi_model_step_plan(const ptmi_model_t *m) { return m ? m->step_plan : -1; }

extern "C" int ptmi_model_step_stamps(ptmi_model_t *m, uint64_t *out, size_t n, int *n_stamps, int *n_wg) {
    if (!m || !n_stamps || !n_wg) return set_error(PTMI_ERR_ARG, "NULL argument");
    *n_stamps = m->step_n_stamps;
    *n_wg = m->step_nb;
    if (!m->step_stamps) return set_error(PTMI_ERR_STATE, "no stage stamps: create the model with PTMI_STEP_STAMPS=1");
    const size_t need = (size_t)m->step_nb * m->step_n_stamps;
    if (!out || n < need) return set_error(PTMI_ERR_ARG, "stamp buffer holds %zu of %zu words", n, need);
    PTMI_HIP(hipStreamSynchronize(lib_stream()));
    PTMI_HIP(hipMemcpy(out, m->step_stamps, need * sizeof(uint64_t), hipMemcpyDeviceToHost));
    return PTMI_OK;
}
