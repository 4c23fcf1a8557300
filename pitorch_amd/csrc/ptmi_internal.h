// Internal declarations shared by the libptmi translation units.
// All device code targets gfx950 (CDNA4, wave64).  Built with
// -ffp-contract=off: every a*b+c below rounds twice unless written as an
// explicit fmaf, which keeps the non-matvec ops bit-compatible with the
// reference's host build.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/ptmi.h"

namespace ptmi {

// ── device math: the reference's libm-free polynomials ──────────────────
// pitorch/ops/core/pt_math.c (same literals and evaluation order).
__device__ __forceinline__ float bits_f(uint32_t u) { return __uint_as_float(u); }

__device__ __forceinline__ float d_expf(float x) {       // pt_math.c:8-25
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
    return poly * bits_f((uint32_t)(n + 127) << 23);
}

__device__ __forceinline__ float d_logf(float x) {       // pt_math.c:31-44
    if (x <= 0.0f) return -3.4028235e+38f;
    uint32_t u = __float_as_uint(x);
    int e = (int)((u >> 23) & 0xFF) - 127;
    float m = bits_f((u & 0x007FFFFFu) | 0x3F800000u);
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

__device__ __forceinline__ float d_wrap_pi(float x) {    // pt_math.c:52-62
    float k = x * 0.15915494309190f;
    k = (float)(int)(k + (k >= 0 ? 0.5f : -0.5f));
    return x - k * 6.28318530717959f;
}

__device__ __forceinline__ float d_sinf(float x) {       // pt_math.c:64-74
    const float pi = 3.14159265358979f, half_pi = 1.57079632679490f;
    x = d_wrap_pi(x);
    if (x > half_pi) x = pi - x;
    else if (x < -half_pi) x = -pi - x;
    float z = x * x;
    float s = -0.00019841270f + z * 0.00000275573f;
    s = 0.00833333333f + z * s;
    s = -0.16666666667f + z * s;
    s = 1.0f + z * s;
    return x * s;
}

__device__ __forceinline__ float d_cosf(float x) {       // pt_math.c:76-87
    const float pi = 3.14159265358979f, half_pi = 1.57079632679490f;
    x = d_wrap_pi(x);
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

__device__ __forceinline__ float d_sqrtf(float x) {      // pt_math.c:92-102
    if (x <= 0.0f) return 0.0f;
    float y = bits_f(0x1fbd1df5u + (__float_as_uint(x) >> 1));
    y = 0.5f * (y + x / y);
    y = 0.5f * (y + x / y);
    y = 0.5f * (y + x / y);
    return y;
}

// RoPE angle for element pair starting at i (pt_ops.c:33-40).
__device__ __forceinline__ void d_rope_cs(int i, int head_dim, int pos, float *c, float *s) {
    int hi = i % head_dim;
    float freq = d_expf(-9.210340372f * (float)hi / (float)head_dim);
    float ang = (float)pos * freq;
    *c = d_cosf(ang);
    *s = d_sinf(ang);
}

// ── cross-lane reductions (wave64) ──────────────────────────────────────
// All-reduce over aligned groups of G lanes, every step a VALU cross-lane
// move: within a row of 16 lanes DPP quad xor 1, quad xor 2, the half-row
// mirror (lane i <-> 7-i: the two quads of an 8-lane group) and the row
// mirror (i <-> 15-i: the two halves of a row); across rows the gfx950
// permlane swaps, which hand every lane both values of the row pair (16)
// or wave half pair (32).
__device__ __forceinline__ float dpp_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_hmirror(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_mirror(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));
}
// Lane l's value and lane l^16's (pl16) or l^32's (pl32), as (lower row or
// half first, upper second) in every lane: v_permlane16_swap /
// v_permlane32_swap of v with itself.
struct LanePair { float lo, hi; };
__device__ __forceinline__ LanePair pl16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    return {__int_as_float(r[0]), __int_as_float(r[1])};
}
__device__ __forceinline__ LanePair pl32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    return {__int_as_float(r[0]), __int_as_float(r[1])};
}
__device__ __forceinline__ int pl16i(int v, int &hi) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    hi = r[1];
    return r[0];
}
__device__ __forceinline__ int pl32i(int v, int &hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    hi = r[1];
    return r[0];
}
// (value, index) argmax step: the larger value, ties to the smaller index
// (pt_ops.c:65-70 keeps the first index of the maximum); NaNs never win.
__device__ __forceinline__ void take_max(float &bv, int &bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}
// Every lane ends with its wave's (value, index) argmax: DPP within rows of
// 16 (quad xor 1, quad xor 2, half-row mirror, row mirror), then the
// permlane swaps across rows and halves (the step is symmetric, so any
// pairing of lanes gives the same result).
__device__ __forceinline__ void wave_argmax(float &bv, int &bi) {
#define PTMI_DPP_TAKE(ctrl)                                                                               \
    take_max(bv, bi, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(bv), ctrl, 0xF, 0xF, true)), \
             __builtin_amdgcn_mov_dpp(bi, ctrl, 0xF, 0xF, true))
    PTMI_DPP_TAKE(0xB1);
    PTMI_DPP_TAKE(0x4E);
    PTMI_DPP_TAKE(0x141);
    PTMI_DPP_TAKE(0x140);
#undef PTMI_DPP_TAKE
    int ih;
    int il = pl16i(bi, ih);
    LanePair p = pl16(bv);
    bv = p.lo; bi = il;
    take_max(bv, bi, p.hi, ih);
    il = pl32i(bi, ih);
    p = pl32(bv);
    bv = p.lo; bi = il;
    take_max(bv, bi, p.hi, ih);
}
// v + (lane l^16's v), v + (lane l^32's v)
__device__ __forceinline__ float xsum16(float v) { const LanePair p = pl16(v); return p.lo + p.hi; }
__device__ __forceinline__ float xsum32(float v) { const LanePair p = pl32(v); return p.lo + p.hi; }

template <int G>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp_xor1(v);
    if constexpr (G >= 4) v += dpp_xor2(v);
    if constexpr (G >= 8) v += dpp_hmirror(v);
    if constexpr (G >= 16) v += dpp_mirror(v);
    if constexpr (G >= 32) v = xsum16(v);
    if constexpr (G >= 64) v = xsum32(v);
    return v;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (G >= 2) v = fmaxf(v, dpp_xor1(v));
    if constexpr (G >= 4) v = fmaxf(v, dpp_xor2(v));
    if constexpr (G >= 8) v = fmaxf(v, dpp_hmirror(v));
    if constexpr (G >= 16) v = fmaxf(v, dpp_mirror(v));
    if constexpr (G >= 32) { const LanePair p = pl16(v); v = fmaxf(p.lo, p.hi); }
    if constexpr (G >= 64) { const LanePair p = pl32(v); v = fmaxf(p.lo, p.hi); }
    return v;
}

// Makes the kernel-argument loads of `v...` complete here, in one batch.
// Without it the compiler fetches kernel arguments lazily, per branch, and
// a kernel that first tests one argument (a prefetch-block split) pays two
// serial scalar round trips before its first vector load.
template <typename T>
__device__ __forceinline__ void kernarg_pin(T v) {
    asm volatile("" ::"s"(v));
}
template <typename... T>
__device__ __forceinline__ void kernarg_batch(T... v) {
    (kernarg_pin(v), ...);
}

// ── matvec launch description ───────────────────────────────────────────
enum Prologue { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_EMBED_RMSNORM = 2, PRO_ATTN_COMBINE = 3 };
constexpr int kMaxCombineDim = 4096;   // PRO_ATTN_COMBINE: x staged in LDS
constexpr int kMaxCombineHeads = 64;
constexpr int kMaxAttnChunks = 8;      // attention chunks per head
enum Epilogue { EPI_STORE = 0, EPI_RESIDUAL = 1, EPI_QKV_ROPE = 2, EPI_SWIGLU = 3 };

// Prefetch of a later stage's weights into L2, XCD by XCD: the rows that
// blocks on XCD x will read in the consumer kernel (its row stripe x) are
// loaded by extra blocks of the producer kernel that run on XCD x.
// Workgroup b runs on XCD b % 8 (round-robin dispatch).
struct PrefetchDesc {
    const float *base;     // consumer weights, rows of row_floats floats
    long row_floats;
    int rows;              // consumer rows
    int stripe;            // consumer rows per XCD stripe
    int blocks;            // prefetch blocks (multiple of 8), 0 = none
    int first_block;       // blockIdx.x of the first prefetch block
    float *sink;           // never written in practice; keeps loads live
};

// Rows of one matvec per XCD stripe and per wave (shared by the launcher
// and by producers that prefetch for it).
// lpr lanes per row, it float4 of x per lane, rows_per_wave rows per wave
// taken np passes of 64/lpr rows at a time (np = 1 or 2), wpb waves per
// block, blocks_per_xcd blocks on each XCD's stripe of rows (linear = 0) or
// 8*blocks_per_xcd blocks over the rows in order (linear = 1).
struct MatvecGeom {
    int lpr, it, np, step, stripe, rows_per_wave, blocks_per_xcd, wpb;
    int linear;            // 1: wave w takes rows [w*rows_per_wave, ...) of the whole matrix
};
bool matvec_geometry(int rows, int n, int pro, int epi, MatvecGeom *g);

// Describe a prefetch of consumer matvec (W rows x ld, with the given
// prologue/epilogue) for a producer whose own blocks end at `first_block`
// and run `producer_threads` threads each.
PrefetchDesc prefetch_for(const float *W, long ld, int rows, int n, int pro, int epi, int first_block,
                          int producer_threads, float *sink);
// Geometry of the matvec the launcher will run for this shape and fusion.
int matvec_compute_blocks(int rows, int n, int pro, int epi);
int matvec_block_threads(int rows, int n, int pro, int epi);

struct MatvecParams {
    const float *W;        // row r starts at W + r*ld
    long ld;               // row stride in floats
    int rows, n;           // output rows, dot length
    const float *x;        // input vector (PRO_EMBED_RMSNORM: embedding table)
    float *y;              // output (EPI_RESIDUAL: residual updated in place)
    int pro;
    const float *norm_w;   // RMSNorm weight [n]
    const int *token;      // PRO_EMBED_RMSNORM: row of x to use (device scalar)
    float *x_out;          // PRO_EMBED_RMSNORM: raw embedding row written here
    int epi;
    const int *pos;        // EPI_QKV_ROPE: decode position (device scalar)
    int q_rows, kv_rows, head_dim;
    float *k_cache, *v_cache;   // this layer's [seq_len, kv_rows] caches
    // PRO_ATTN_COMBINE: x = softmax-combined attention partials of all heads
    const float *att_o;    // [heads][chunks][head_dim] unnormalised sums
    const float *att_ml;   // [heads][chunks][2] (chunk max, chunk sum)
    int att_chunks, att_chunk, att_heads;
    int rows_per_wave;     // filled by the launcher
    int stripe, blocks_per_xcd, linear;
    PrefetchDesc pf;       // optional L2 prefetch for the next stage
};

// Prefetch blocks' body (any kernel): loads its share of stripe
// (blockIdx.x % 8) of the consumer weights and discards it.
__device__ __forceinline__ void run_prefetch(const PrefetchDesc &pf) {
    kernarg_batch(pf.base, pf.row_floats, pf.rows, pf.stripe, pf.blocks, pf.first_block, pf.sink, (int)blockDim.x);
    const int q = (int)blockIdx.x - pf.first_block;
    const int xcd = (int)(blockIdx.x & 7), rank = q >> 3, per_xcd = pf.blocks >> 3;
    const long r0 = (long)xcd * pf.stripe;
    const long r1 = r0 + pf.stripe < (long)pf.rows ? r0 + pf.stripe : (long)pf.rows;
    if (r0 >= r1) return;
    const long f0 = r0 * pf.row_floats / 4, f1 = r1 * pf.row_floats / 4;
    const long chunk = (f1 - f0 + per_xcd - 1) / per_xcd;
    const long a = f0 + rank * chunk;
    const long e = a + chunk < f1 ? a + chunk : f1;
    const float4 *src = reinterpret_cast<const float4 *>(pf.base);
    float acc = 0.0f;
    const long step = (long)blockDim.x * 8;
    for (long i = a + threadIdx.x; i < e; i += step) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const long j = i + (long)u * blockDim.x;
            v[u] = src[j < e ? j : e - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) acc += v[u].x;
    }
    if (acc == -1.2345e-37f) pf.sink[0] = acc;
}

// Kernel launch, optionally bracketed by HIP events that the command
// processor timestamps at the kernel's own start and end (profiling).
template <typename F, typename... A>
inline void launch_k(F f, dim3 g, dim3 b, size_t shmem, hipStream_t s, hipEvent_t e0, hipEvent_t e1, A... a) {
    if (e0) hipExtLaunchKernelGGL(f, g, b, (uint32_t)shmem, s, e0, e1, 0, a...);
    else hipLaunchKernelGGL(f, g, b, shmem, s, a...);
}

// Launch y = epilogue(W . prologue(x)); validates shapes, picks a kernel.
// x_reread: the ablation kernel that re-reads x for every row pass.
int launch_matvec(MatvecParams p, hipStream_t s, hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr,
                  bool x_reread = false);

// Split-K partial sums left in the workspace for the next kernel to add up
// (dense [splits][M][N]; C = (Cin +) sum over z ascending of parts[z]).
struct SplitK {
    const float *parts;
    int splits;            // 0: C was written by the GEMM itself
    long stride;           // M*N
};

// sum_z parts[z*stride + idx] for z = 0..splits-1 in ascending order (the
// split-K reduction).  Loads go out eight at a time before any is added,
// so a reduction costs about splits/8 memory round trips, not splits.
__device__ __forceinline__ float sum_splits(const float *parts, int splits, long stride, long idx) {
    float v = 0.0f;
    for (int z0 = 0; z0 < splits; z0 += 8) {
        float pv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) pv[u] = parts[(long)min(z0 + u, splits - 1) * stride + idx];
#pragma unroll
        for (int u = 0; u < 8; u++) v = z0 + u < splits ? v + pv[u] : v;
    }
    return v;
}

// Element-wise epilogues fused into an NT GEMM (whole K, no split):
//  GEMM_EPI_ROPE: RoPE at position m on columns [0, 2*rope_dim) (q then k),
//    applied to C in place;
//  GEMM_EPI_SWIGLU: C columns (2i, 2i+1) hold (h1, h3); also writes
//    out[m*ld + i] = (h1*sigmoid(h1))*h3.
//  GEMM_EPI_SWIGLU_BWD (NN GEMM): C[m][i] is d_sh; with (h1, h3) =
//    aux[m*aux_ld + 2i + {0,1}] it writes d_h1, d_h3 to out[m*ld + 2i + {0,1}]
//    and silu(h1)*h3 to out2[m*ld2 + i]; C itself is not stored.
enum { GEMM_EPI_NONE = 0, GEMM_EPI_ROPE = 1, GEMM_EPI_SWIGLU = 2, GEMM_EPI_SWIGLU_BWD = 3 };
struct GemmEpi {
    int kind;
    float *out;            // SWIGLU / SWIGLU_BWD output
    long ld;               // its row stride
    int rope_dim, head_dim;
    float *out2;           // SWIGLU_BWD: recomputed silu(h1)*h3
    long ld2;
    const float *aux;      // SWIGLU_BWD: the forward's (h1, h3) pairs
    long aux_ld;
};

// RMSNorm (pt_ops.c:5-12) fused into the A operand of an NT GEMM with a
// fused epilogue (whole K = the row length, 32x32 tiles, float4 rows):
// C = epi(diag(inv) . (X . diag(w)) . B^T), inv[m] = 1/sqrt(mean_k x[m][k]^2
// + 1e-5), where the rows X are
//   PLAIN:  A itself;
//   SPLITS: cin + the pending split-K partial sums pk (at most kNormSplits);
//   EMBED:  emb[tok[m]] (and tok_bits marks the tokens of rows < M-1).
// The blocks of each row tile also store, each a share of the columns, X
// to x_out (SPLITS, EMBED) and the normalized rows x * inv * w to xn_out, as
// the standalone RMSNorm kernel does.  Every row array has leading
// dimension K.
enum { GEMM_NORM_PLAIN = 1, GEMM_NORM_SPLITS = 2, GEMM_NORM_EMBED = 3 };
constexpr int kNormSplits = 4;
struct GemmNorm {
    int kind;              // 0: no fused norm
    const float *w;        // norm weights [K]
    SplitK pk;             // SPLITS
    const float *cin;      // SPLITS: residual addend (may be null)
    const int *tok;        // EMBED
    const float *emb;
    unsigned *tok_bits;
    float *x_out;          // SPLITS, EMBED: the completed rows
    float *xn_out;         // the normalized rows
};
// Whether launch_gemm fuses the norm nm into the NT GEMM [M,N,K] with A
// rows of stride lda, B = W [N][K] (stride ldb) and epilogue `epi_kind`
// (else the caller runs the norm, then the GEMM).
bool gemm_norm_fusable(int M, int N, int K, const float *A, long lda, const float *B, long ldb, int epi_kind,
                       const GemmNorm &nm);

// C[M,N] (+)= op(A).op(B) on the matrix cores; op 0 NN, 1 TN (A stored
// [K][M]), 2 NT (B stored [N][K]).  ws: split-K workspace (may be null).
// With accumulate, Cin (same leading dimension as C; null = C itself) is
// the addend: C = Cin + op(A).op(B).  With `defer`, a split-K GEMM skips its
// reduction launch and leaves the partials to the caller (defer->splits > 0;
// C is then not written); otherwise defer->splits = 0.
int launch_gemm(int op, const float *A, long lda, const float *B, long ldb, float *C, long ldc, int M, int N,
                int K, int accumulate, float *ws, size_t ws_floats, hipStream_t s, const float *Cin = nullptr,
                SplitK *defer = nullptr, const GemmEpi *epi = nullptr, const GemmNorm *norm = nullptr);

// Workspace floats launch_gemm needs to split this GEMM's K the way it does
// with a workspace of ws_floats floats (0: no split).
size_t gemm_workspace_floats(int op, int M, int N, int K, size_t ws_floats);

// Grouped C[M,N] = A^T.B GEMMs (TN; A stored [K][M]; C written, not
// accumulated), one launch of 32x32 tiles over all of them.  prepare fills host_desc (gemm_group_desc_bytes(n)
// bytes); the caller copies it to device memory for the launch.
// upd != null: the SGD step of the weight whose gradient C is, fused into
// the epilogue: upd[m][n] -= *lr * C[m][n] (same layout as C), except rows
// m whose bit is set in keep (their gradient is completed, and the weight
// updated, by a later kernel).
struct TnGemm {
    const float *A; long lda;
    const float *B; long ldb;
    float *C; long ldc;
    int M, N, K;
    float *upd = nullptr;
    const unsigned *keep = nullptr;
};
size_t gemm_group_desc_bytes(int n);
int gemm_tn_group_prepare(const TnGemm *list, int n, const float *lr, void *host_desc, int *tiles_total, int *vec);
// Entries [i0, i1) of a prepared table, whose tiles number `tiles`.
int launch_gemm_tn_group(const void *dev_desc, int i0, int i1, int tiles, int vec, hipStream_t s);

// ── library state ───────────────────────────────────────────────────────
struct Config {
    int dim, hidden, n_layers, n_heads, n_kv_heads, vocab, seq_len;
    int head_dim, kv_dim, shared;
};

// Device copy of one registered blob in the device layout.
struct Resident {
    const char *blob;          // host blob (header included)
    size_t bytes;
    int32_t header[7];         // the 28-byte header as registered
    int explicit_holds;        // ptmi_register_weights calls not yet unregistered
    int model_holds;           // live models created over this blob
    Config c;
    float *mem;                // one allocation for all tensors
    size_t mem_floats;
    float *emb, *rms_att, *wqkv, *wo, *rms_ffn, *w13, *w2, *rms_final, *wcls;
    // host tensor offsets in floats from blob+28 (file order)
    size_t off_emb, off_rms_att, off_wq, off_wk, off_wv, off_wo, off_rms_ffn,
           off_w1, off_w2, off_w3, off_rms_final, off_wcls, off_end;
};

int  set_error(int status, const char *fmt, ...);
int  ensure_init();
hipStream_t lib_stream();
bool lib_initialised();
int  lib_device();
// Locates ptmi_gemm_dev_noalloc's fixed device scratch on `device` (the
// current device); called once per device by ptmi_init.
int  gemm_scratch_setup(int device);
int  hip_check(hipError_t e, const char *what);
Resident *find_resident(const void *p);
// Registration holds: register_blob takes one (explicit = ptmi_register_weights,
// else a model's), release_blob drops a model's; the device copy is freed
// when no hold is left.
Resident *register_blob(const void *blob, size_t bytes, bool explicit_hold, int *status);
void release_blob(Resident *r);
int  upload_resident(Resident *r, hipStream_t s);   // host blob -> device layout
int  download_resident(Resident *r, void *blob, hipStream_t s);
int  parse_config(const void *blob, size_t bytes, Config *c);
// Grow-only device scratch owned by the library (host-pointer entry points).
float *scratch_buf(int slot, size_t floats);

}  // namespace ptmi

#define PTMI_HIP(call)                                              \
    do {                                                            \
        hipError_t e_ = (call);                                     \
        if (e_ != hipSuccess) return ptmi::hip_check(e_, #call);    \
    } while (0)
