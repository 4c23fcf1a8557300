// fp32 matvec y = W[rows, n] . x[n] for gfx950, with the decode step's
// prologues (RMSNorm, embedding gather) and epilogues (residual add,
// RoPE + KV-cache write, SwiGLU) fused in.
//
// HBM-bound design (2 flop per 4-byte weight, ~0.5 flop/B):
//  * LPR lanes own one row; each lane streams 16-byte (dwordx4) weight
//    chunks sub, sub+LPR, ... so a wave's load instruction covers 64/LPR
//    rows x LPR*16 contiguous bytes — fully used 64..1024-byte segments.
//  * The lane's x chunks (at most 9 float4) stay in registers for the whole
//    wave: x is read once per wave, never re-staged per row.
//  * Two row passes are issued before either is reduced so each lane keeps
//    2*IT independent 16-byte loads in flight.
//  * Row sums are combined with DPP / permlane cross-lane moves (no LDS tree);
//    LDS holds only the <=64 finished row values a wave hands to its
//    epilogue.
// Reduction order differs from the reference's sequential j loop
// (pitorch/ops/core/pt_ops.c:72-80): results agree to fp32 rounding.
#include "ptmi_internal.h"

#include <algorithm>

namespace ptmi {

namespace {

constexpr int kWaves = 4;          // waves per workgroup
constexpr int kMaxRowsPerWave = 64;
constexpr int kBigRows = 16384;    // matrices with at least this many rows ...
constexpr int kBigWaves = 8192;    // ... run about this many single-iteration waves

// v if keep, else 0 (branch-free per-lane select)
__device__ __forceinline__ float4 sel4(bool keep, float4 v) {
    return make_float4(keep ? v.x : 0.0f, keep ? v.y : 0.0f, keep ? v.z : 0.0f, keep ? v.w : 0.0f);
}

__device__ __forceinline__ float dot4(float4 w, float4 x, float acc) {
    acc = fmaf(w.x, x.x, acc);
    acc = fmaf(w.y, x.y, acc);
    acc = fmaf(w.z, x.z, acc);
    acc = fmaf(w.w, x.w, acc);
    return acc;
}

// Epilogue for rows [row0, row0 + nrows) whose sums sit in vals[0..nrows).
// Runs on one wave; lane i handles row row0+i (pairs handled by even lanes).
// EPI_RESIDUAL: `res` is y[row0 + lane], loaded in the prologue.
template <int EPI>
__device__ __forceinline__ void run_epilogue(const MatvecParams &p, const float *vals,
                                             int row0, int nrows, int lane, int pos, float res) {
    if (lane >= nrows) return;
    const int r = row0 + lane;
    const float v = vals[lane];
    if constexpr (EPI == EPI_STORE) {
        p.y[r] = v;
    } else if constexpr (EPI == EPI_RESIDUAL) {   // vec_add(x, x, xb2): llama2.c:180,190
        p.y[r] = res + v;
    } else if constexpr (EPI == EPI_SWIGLU) {     // rows interleaved w1[i], w3[i]
        if (lane & 1) return;                     // llama2.c:187-188 (silu, vec_mul)
        const float h1 = v, h3 = vals[lane + 1];
        const float s = h1 / (1.0f + d_expf(-h1));
        p.y[r >> 1] = s * h3;
    } else {                                      // rope + KV write: llama2.c:147-151
        static_assert(EPI == EPI_QKV_ROPE, "epilogue");
        if (lane & 1) return;
        const float a = v, b = vals[lane + 1];
        if (r < p.q_rows) {
            float c, s;
            d_rope_cs(r, p.head_dim, pos, &c, &s);
            p.y[r] = a * c - b * s;
            p.y[r + 1] = a * s + b * c;
        } else if (r < p.q_rows + p.kv_rows) {
            const int i = r - p.q_rows;
            float c, s;
            d_rope_cs(i, p.head_dim, pos, &c, &s);
            float *dst = p.k_cache + (long)pos * p.kv_rows + i;
            dst[0] = a * c - b * s;
            dst[1] = a * s + b * c;
        } else {
            const int i = r - p.q_rows - p.kv_rows;
            float *dst = p.v_cache + (long)pos * p.kv_rows + i;
            dst[0] = a;
            dst[1] = b;
        }
    }
}

// Register-resident-x kernel: LPR lanes per row, IT float4 chunks per lane,
// NP passes of 64/LPR rows loaded together.  IT = ceil(n/4 / LPR), so only
// the last chunk can run past the row: its address is clamped into the row
// and its value replaced by 0, which keeps every load unconditional.
//
// XR (ablation, plain y = Wx only): x is re-read from memory for every row
// pass instead of once per wave — the MI355X counterpart of the reference's
// smatvec_tmu_no_packing baseline (pitorch/ops/matvec/matvec_no_packing.c:
// 1-10), which re-packs x for every dispatch.
template <int LPR, int IT, int NP, int PRO, int EPI, bool XR = false>
__global__ __launch_bounds__(256) void k_matvec(MatvecParams p) {
    static_assert(!XR || (PRO == PRO_NONE && EPI == EPI_STORE), "the x re-read ablation is a plain matvec");
    constexpr int RPP = 64 / LPR;                  // rows per pass
    constexpr bool kNorm = PRO == PRO_RMSNORM || PRO == PRO_EMBED_RMSNORM;
    __shared__ float ybuf[kWaves][kMaxRowsPerWave];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int slot = lane / LPR;
    const int sub = lane % LPR;
    const int n4 = p.n >> 2;
    // The decode position: a scalar load issued before anything else (it
    // stays a scalar load only ahead of the asm statements below).
    int pos = 0;
    if constexpr (EPI == EPI_QKV_ROPE || PRO == PRO_ATTN_COMBINE) pos = *p.pos;
    // The compute path's launch parameters are fetched in the same batch
    // as the prefetch test below; otherwise every wave pays a second
    // kernel-argument round trip after the branch.
    kernarg_batch(p.W, p.x, p.ld, p.rows, p.n, p.stripe, p.rows_per_wave, p.linear, (int)blockDim.x);
    if constexpr (kNorm) kernarg_batch(p.norm_w);
    if constexpr (EPI == EPI_RESIDUAL) kernarg_batch(p.y);
    if constexpr (PRO == PRO_EMBED_RMSNORM) kernarg_batch(p.token);
    if constexpr (PRO == PRO_ATTN_COMBINE) kernarg_batch(p.att_o, p.att_ml, p.att_chunks, p.att_heads);
    // Blocks past the compute grid prefetch the next stage's weights.
    if ((int)blockIdx.x >= 8 * p.blocks_per_xcd) {
        run_prefetch(p.pf);
        return;
    }
    // XCD-striped rows: block b (on XCD b%8) works inside stripe b%8; or
    // rows in block order over the whole matrix.
    const int wpb = blockDim.x >> 6;
    const bool lin = p.linear != 0;                    // uniform
    const long s0 = lin ? 0L : (long)(blockIdx.x & 7) * p.stripe;
    const long s1 = lin ? (long)p.rows : (s0 + p.stripe < (long)p.rows ? s0 + p.stripe : (long)p.rows);
    const long row0l = s0 + ((long)(lin ? blockIdx.x : blockIdx.x >> 3) * wpb + wave) * p.rows_per_wave;
    const bool active = row0l < s1;
    const int row0 = active ? (int)row0l : 0;
    const int nrows = active ? (int)min((long)p.rows_per_wave, s1 - row0l) : 0;

    // Weight loads of the NP passes starting at row `base` of the wave.
    // Rows past the end re-read the wave's last row; their sums are dropped.
    constexpr int kIterRows = NP * RPP;
    float4 wv[NP][IT];
    // Weight rows are read with nontemporal loads: each is read once per
    // step, and the hint keeps this stream from evicting the weights that
    // prefetch blocks have staged in L2 for the next kernels (decode
    // 3498 -> 3565 tok/s, stories110M).
    typedef float fx4 __attribute__((ext_vector_type(4)));
    auto load_rows = [&](int base) {
#pragma unroll
        for (int q = 0; q < NP; q++) {
            const int r = max(0, min(base + q * RPP + slot, nrows - 1));   // idle waves read row 0
            const fx4 *w = reinterpret_cast<const fx4 *>(p.W + (long)(row0 + r) * p.ld);
#pragma unroll
            for (int it = 0; it < IT; it++) {
                const int c = sub + it * LPR;
                const fx4 t = __builtin_nontemporal_load(w + (it < IT - 1 ? c : min(c, n4 - 1)));
                wv[q][it] = make_float4(t.x, t.y, t.z, t.w);
            }
        }
    };
    // This lane's x chunks (and RMSNorm weights).
    float4 xr[IT], nw[IT];
    auto load_x = [&](const float *src) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int c = sub + it * LPR;
            const int cc = it < IT - 1 ? c : min(c, n4 - 1);
            xr[it] = reinterpret_cast<const float4 *>(src)[cc];
            if constexpr (kNorm) nw[it] = reinterpret_cast<const float4 *>(p.norm_w)[cc];
        }
    };

    // ---- issue order.  Loads return in issue order, so a loaded value is
    // usable only once every load issued before it has returned.  The
    // prologue's few loads go out first and the weight stream right behind
    // them: the prologue arithmetic then waits for its own round trip while
    // the weights are in flight.  The embedding row's address needs the
    // token id, so that prologue issues its x loads after the weights.  A
    // plain y = Wx has no prologue arithmetic; there the weights go first
    // (measured faster on the large classifier-shaped matrices).
    constexpr bool kXFirst = !(PRO == PRO_NONE && EPI == EPI_STORE);
    // PRO_ATTN_COMBINE inputs: the active chunks' partial sums and
    // statistics (the slots past them re-read the last active chunk, the same
    // cache lines, and are dropped later by selects; att_chunk >= 1).
    constexpr int kFastI = 6;                            // n <= 6 * threads in one round trip
    float ov[kFastI][kMaxAttnChunks], mv[kMaxAttnChunks], lv[kMaxAttnChunks];
    const int nthr = blockDim.x;
    const int hd = PRO == PRO_ATTN_COMBINE ? p.n / p.att_heads : 1;
    const int nch = p.att_chunks;
    const bool fast = p.n <= kFastI * nthr;              // uniform
    if constexpr (PRO == PRO_ATTN_COMBINE) {
        if (fast) {
#pragma unroll
            for (int k = 0; k < kFastI; k++) {
                if (k * nthr >= p.n) break;              // uniform: slots past n load nothing
                const int i = min((int)threadIdx.x + k * nthr, p.n - 1);
                const int h = i / hd, d = i - h * hd;
                const float *o = p.att_o + (long)h * nch * hd + d;
#pragma unroll
                for (int c = 0; c < kMaxAttnChunks; c++) ov[k][c] = o[(long)min(c, min(nch, pos / p.att_chunk + 1) - 1) * hd];
            }
        }
        const int h_ml = min((int)threadIdx.x, p.att_heads - 1);
        const float *ml = p.att_ml + 2L * h_ml * nch;
#pragma unroll
        for (int c = 0; c < kMaxAttnChunks; c++) {
            const int cc = min(c, min(nch, pos / p.att_chunk + 1) - 1);
            mv[c] = ml[2 * cc];
            lv[c] = ml[2 * cc + 1];
        }
    } else if constexpr (kXFirst) {
        load_x(p.x);
    }
    __builtin_amdgcn_sched_barrier(0);            // keep the issue order above
    load_rows(0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PRO == PRO_EMBED_RMSNORM) load_x(p.x + (long)(*p.token) * p.n);
    if constexpr (PRO == PRO_NONE && !kXFirst && !XR) load_x(p.x);
    // The residual this wave's epilogue adds to (its rows only).
    float res = 0.0f;
    if constexpr (EPI == EPI_RESIDUAL) {
        if (lane < nrows) res = p.y[row0 + lane];
    }

    // ---- prologue arithmetic
    if constexpr (PRO == PRO_ATTN_COMBINE) {
        // x[i] = sum_c w[h][c] o_c[i], w[h][c] = e^(m_c - M) / sum_c' l_c' e^(m_c' - M)
        // over the active chunks of head h = i/hd, once per workgroup into LDS.
        __shared__ float xcomb[kMaxCombineDim];
        __shared__ float wts[kMaxCombineHeads][kMaxAttnChunks];
        const int active = pos / p.att_chunk + 1;
        if ((int)threadIdx.x < p.att_heads) {
            float M = mv[0];
#pragma unroll
            for (int c = 1; c < kMaxAttnChunks; c++) M = c < active ? fmaxf(M, mv[c]) : M;
            float f[kMaxAttnChunks], L = 0.0f;
#pragma unroll
            for (int c = 0; c < kMaxAttnChunks; c++) {
                f[c] = c < active ? d_expf(mv[c] - M) : 0.0f;
                L = c < active ? fmaf(lv[c], f[c], L) : L;
            }
            const float inv = 1.0f / L;
#pragma unroll
            for (int c = 0; c < kMaxAttnChunks; c++) wts[threadIdx.x][c] = f[c] * inv;
        }
        __syncthreads();
        if (fast) {
#pragma unroll
            for (int k = 0; k < kFastI; k++) {
                if (k * nthr >= p.n) break;
                const int i = (int)threadIdx.x + k * nthr;
                if (i < p.n) {
                    const int h = i / hd;
                    float v = 0.0f;
#pragma unroll
                    for (int c = 0; c < kMaxAttnChunks; c++) v = c < active ? fmaf(ov[k][c], wts[h][c], v) : v;
                    xcomb[i] = v;
                }
            }
        } else {
            for (int i = threadIdx.x; i < p.n; i += nthr) {
                const int h = i / hd, d = i - h * hd;
                const float *o = p.att_o + (long)h * nch * hd + d;
                float ovs[kMaxAttnChunks];
#pragma unroll
                for (int c = 0; c < kMaxAttnChunks; c++) ovs[c] = o[(long)min(c, nch - 1) * hd];
                float v = 0.0f;
#pragma unroll
                for (int c = 0; c < kMaxAttnChunks; c++) v = c < active ? fmaf(ovs[c], wts[h][c], v) : v;
                xcomb[i] = v;
            }
        }
        __syncthreads();
        load_x(xcomb);
    }
    // The last chunk past the row contributes 0 (x and w both zeroed, so
    // a non-finite weight read through the clamped address cannot leak in).
    const bool tail_in = sub + (IT - 1) * LPR < n4;
    if constexpr (!XR) xr[IT - 1] = sel4(tail_in, xr[IT - 1]);
    if (PRO == PRO_EMBED_RMSNORM && blockIdx.x == 0 && wave == 0 && slot == 0) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int c = sub + it * LPR;
            if (c < n4) reinterpret_cast<float4 *>(p.x_out)[c] = xr[it];
        }
    }
    if constexpr (kNorm) {                        // rmsnorm, pt_ops.c:5-12
        float ss = 0.0f;
#pragma unroll
        for (int it = 0; it < IT; it++)
            ss += xr[it].x * xr[it].x + xr[it].y * xr[it].y + xr[it].z * xr[it].z + xr[it].w * xr[it].w;
        ss = group_sum<LPR>(ss);
        const float inv = 1.0f / d_sqrtf(ss / (float)p.n + 1e-5f);
#pragma unroll
        for (int it = 0; it < IT; it++) {
            xr[it].x = xr[it].x * inv * nw[it].x;
            xr[it].y = xr[it].y * inv * nw[it].y;
            xr[it].z = xr[it].z * inv * nw[it].z;
            xr[it].w = xr[it].w * inv * nw[it].w;
        }
    }

    for (int base = 0; base < nrows; base += kIterRows) {
        if (base > 0) load_rows(base);
        if constexpr (XR) {
            // a fresh read of x for this pass's rows; the barrier keeps the
            // compiler from hoisting the loop-invariant loads out of the loop
            asm volatile("" ::: "memory");
            load_x(p.x);
            xr[IT - 1] = sel4(tail_in, xr[IT - 1]);
        }
#pragma unroll
        for (int q = 0; q < NP; q++) {
            float acc = 0.0f;
#pragma unroll
            for (int it = 0; it < IT; it++)
                acc = dot4(it < IT - 1 ? wv[q][it] : sel4(tail_in, wv[q][it]), xr[it], acc);
            acc = group_sum<LPR>(acc);
            const int r = base + q * RPP + slot;
            if (sub == 0 && r < nrows) ybuf[wave][r] = acc;
        }
    }
    __syncthreads();
    if (active) run_epilogue<EPI>(p, ybuf[wave], row0, nrows, lane, pos, res);
}

// Long rows (n > 64*9*4): one wave per row pair, x read through the cache
// in 64-chunk strides.  Used by the drop-in path for transposed weights
// (e.g. W_cls^T, in_dim = vocab) — not by the decode step.
__global__ __launch_bounds__(256) void k_matvec_long(MatvecParams p) {
    __shared__ float ybuf[kWaves][kMaxRowsPerWave];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n4 = p.n >> 2;
    const long wave_id = (long)blockIdx.x * kWaves + wave;
    const long row0l = wave_id * p.rows_per_wave;
    const bool active = row0l < p.rows;
    const int row0 = active ? (int)row0l : 0;
    const int nrows = active ? min(p.rows_per_wave, p.rows - row0) : 0;
    const float4 *x4 = reinterpret_cast<const float4 *>(p.x);
    for (int r = 0; r < nrows; r += 2) {
        const bool vb = r + 1 < nrows;
        const float4 *wa = reinterpret_cast<const float4 *>(p.W + (long)(row0 + r) * p.ld);
        const float4 *wb = reinterpret_cast<const float4 *>(p.W + (long)(row0 + (vb ? r + 1 : r)) * p.ld);
        float a = 0.0f, b = 0.0f;
        for (int c = lane; c < n4; c += 64) {
            const float4 xv = x4[c];
            a = dot4(wa[c], xv, a);
            b = dot4(wb[c], xv, b);
        }
        a = group_sum<64>(a);
        b = group_sum<64>(b);
        if (lane == 0) {
            ybuf[wave][r] = a;
            if (vb) ybuf[wave][r + 1] = b;
        }
    }
    __syncthreads();
    if (active) run_epilogue<EPI_STORE>(p, ybuf[wave], row0, nrows, lane, 0, 0.0f);
}

// Any alignment / any n: one wave per row, scalar loads.
__global__ __launch_bounds__(256) void k_matvec_scalar(MatvecParams p) {
    const int lane = threadIdx.x & 63;
    const long row = (long)blockIdx.x * kWaves + (threadIdx.x >> 6);
    if (row >= p.rows) return;
    const float *w = p.W + row * p.ld;
    float a = 0.0f;
    for (int j = lane; j < p.n; j += 64) a = fmaf(w[j], p.x[j], a);
    a = group_sum<64>(a);
    if (lane == 0) p.y[row] = (p.epi == EPI_RESIDUAL) ? p.y[row] + a : a;
}

using KernelFn = void (*)(MatvecParams);

template <int LPR, int NP, int PRO, int EPI>
KernelFn pick_it(int it) {
    switch (it) {
    case 1: return k_matvec<LPR, 1, NP, PRO, EPI>;
    case 2: return k_matvec<LPR, 2, NP, PRO, EPI>;
    case 3: return k_matvec<LPR, 3, NP, PRO, EPI>;
    case 4: return k_matvec<LPR, 4, NP, PRO, EPI>;
    case 5: return k_matvec<LPR, 5, NP, PRO, EPI>;
    case 6: return k_matvec<LPR, 6, NP, PRO, EPI>;
    case 7: return k_matvec<LPR, 7, NP, PRO, EPI>;
    case 8: return k_matvec<LPR, 8, NP, PRO, EPI>;
    case 9: return k_matvec<LPR, 9, NP, PRO, EPI>;
    default: return nullptr;
    }
}

// Only the (prologue, epilogue) pairs the library launches are built:
// plain y=Wx, QKV (+embed on layer 0), residual (Wo, w2), SwiGLU (w1|w3),
// classifier (RMSNorm prologue, plain store).
template <int LPR, int NP>
KernelFn pick_role(int it, int pro, int epi) {
    if (pro == PRO_NONE && epi == EPI_STORE) return pick_it<LPR, NP, PRO_NONE, EPI_STORE>(it);
    if (pro == PRO_NONE && epi == EPI_RESIDUAL) return pick_it<LPR, NP, PRO_NONE, EPI_RESIDUAL>(it);
    if (pro == PRO_RMSNORM && epi == EPI_STORE) return pick_it<LPR, NP, PRO_RMSNORM, EPI_STORE>(it);
    if (pro == PRO_RMSNORM && epi == EPI_SWIGLU) return pick_it<LPR, NP, PRO_RMSNORM, EPI_SWIGLU>(it);
    if (pro == PRO_RMSNORM && epi == EPI_QKV_ROPE) return pick_it<LPR, NP, PRO_RMSNORM, EPI_QKV_ROPE>(it);
    if (pro == PRO_EMBED_RMSNORM && epi == EPI_QKV_ROPE)
        return pick_it<LPR, NP, PRO_EMBED_RMSNORM, EPI_QKV_ROPE>(it);
    if (pro == PRO_ATTN_COMBINE && epi == EPI_RESIDUAL) return pick_it<LPR, NP, PRO_ATTN_COMBINE, EPI_RESIDUAL>(it);
    return nullptr;
}

template <int LPR>
KernelFn pick(int it, int np, int pro, int epi) {
    return np == 2 ? pick_role<LPR, 2>(it, pro, epi) : pick_role<LPR, 1>(it, pro, epi);
}

template <int LPR, int NP>
KernelFn pick_xr_np(int it) {
    switch (it) {
    case 1: return k_matvec<LPR, 1, NP, PRO_NONE, EPI_STORE, true>;
    case 2: return k_matvec<LPR, 2, NP, PRO_NONE, EPI_STORE, true>;
    case 3: return k_matvec<LPR, 3, NP, PRO_NONE, EPI_STORE, true>;
    case 4: return k_matvec<LPR, 4, NP, PRO_NONE, EPI_STORE, true>;
    case 5: return k_matvec<LPR, 5, NP, PRO_NONE, EPI_STORE, true>;
    case 6: return k_matvec<LPR, 6, NP, PRO_NONE, EPI_STORE, true>;
    case 7: return k_matvec<LPR, 7, NP, PRO_NONE, EPI_STORE, true>;
    case 8: return k_matvec<LPR, 8, NP, PRO_NONE, EPI_STORE, true>;
    case 9: return k_matvec<LPR, 9, NP, PRO_NONE, EPI_STORE, true>;
    default: return nullptr;
    }
}

template <int LPR>
KernelFn pick_xr(int it, int np) {
    return np == 2 ? pick_xr_np<LPR, 2>(it) : pick_xr_np<LPR, 1>(it);
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// Lanes-per-row so that each lane holds at most 9 float4 of x; rows split
// into 8 XCD stripes (multiples of the row-pair step); rows-per-wave so
// that each XCD runs ~256 waves (8 per CU) when the matrix is big enough.
// Kernel geometry, chosen from measurements on MI355X (graph-replayed
// launches, weights in HBM or MALL):
//  * >= 16384 rows (the classifier), any prologue: many short waves in row
//    order (32000x768: 18.1 vs 19.1 us; 32000x512: 13.1 vs 15.8 us).  A
//    wave that walks several row groups one after another leaves the tail
//    of the launch to a few late waves.
//  * With a prologue (RMSNorm, embedding, attention combine), whose cost is
//    paid per wave or per workgroup: the fewest lanes per row that keep a
//    lane's x slice within 9 float4, two row passes per iteration, ~256
//    waves per XCD (8 per CU), 4 waves per block.  More workgroups make
//    these kernels slower.
//  * Without a prologue: many small workgroups win (768x768: 2.57 vs
//    3.18 us; 2304x768: 3.19 vs 3.64 us).  For rows of >= 192 floats, ~4096
//    single-wave blocks with as many lanes per row as that allows; for
//    shorter rows, ~1024 waves of two-pass rows.
bool matvec_geometry(int rows, int n, int pro, int epi, MatvecGeom *g) {
    const int n4 = n / 4;
    if (n % 4 || n4 > 64 * 9 || rows <= 0) return false;
    const int gran = (epi == EPI_SWIGLU || epi == EPI_QKV_ROPE) ? 2 : 1;   // row pairs stay in one wave
    const int lpr_min = n4 <= 8 * 9 ? 8 : n4 <= 16 * 9 ? 16 : n4 <= 32 * 9 ? 32 : 64;
    const int per = (rows + 7) / 8;
    int lpr = lpr_min, rpw, wpb;
    bool two;
    int linear = 0;
    if (rows >= kBigRows) {
        // Large matrices (the classifier): one iteration per wave, each
        // wave's few rows loaded at once, ~8192 waves of 4, rows in block
        // order.  Lanes per row: the widest power of two that keeps >= 3/4
        // of the lanes' chunks inside the row; then, while there are too
        // many waves, halve it (x slice <= 6 float4), or take two passes,
        // or more rows per wave.
        lpr = 64;
        while (lpr > lpr_min && 4 * n4 < 3 * lpr * ((n4 + lpr - 1) / lpr)) lpr /= 2;
        int it = (n4 + lpr - 1) / lpr;
        int rpp = 64 / lpr;
        two = gran > rpp;
        rpw = two ? 2 * rpp : rpp;
        while ((rows + rpw - 1) / rpw > kBigWaves) {
            if (!two && lpr / 2 >= lpr_min && 2 * it <= 6) {
                lpr /= 2;
                it = (n4 + lpr - 1) / lpr;
                rpp = 64 / lpr;
                rpw = std::max(rpp, gran);
                two = rpw > rpp;
            } else if (!two) {
                two = true;
                rpw = 2 * rpp;
            } else if (rpw < kMaxRowsPerWave) {
                rpw *= 2;
            } else {
                break;
            }
        }
        g->stripe = (per + gran - 1) / gran * gran;
        wpb = kWaves;
        linear = 1;
    } else if (pro != PRO_NONE) {
        const int step = 2 * (64 / lpr);
        g->stripe = (per + step - 1) / step * step;
        rpw = (g->stripe + 255) / 256;
        rpw = (rpw + step - 1) / step * step;
        rpw = std::min(std::max(rpw, step), kMaxRowsPerWave);
        two = true;
        wpb = kWaves;
    } else {
        const int target = n4 > 8 * 9 ? 4096 : 1024;
        rpw = std::max((rows + target - 1) / target, gran);
        while (lpr < 64 && lpr < n4 && 64 / lpr > rpw) lpr *= 2;
        const int rpp = 64 / lpr;
        rpw = std::min(std::max(rpw, rpp), kMaxRowsPerWave);
        rpw = (rpw + gran - 1) / gran * gran;
        two = rpw > rpp;
        g->stripe = (per + gran - 1) / gran * gran;
        const int waves = (g->stripe + rpw - 1) / rpw;
        wpb = n4 > 8 * 9 ? 1 : waves >= 128 ? 4 : waves >= 64 ? 2 : 1;
    }
    g->lpr = lpr;
    g->it = (n4 + lpr - 1) / lpr;
    g->np = two ? 2 : 1;
    g->step = gran;
    g->rows_per_wave = rpw;
    g->linear = linear;
    g->wpb = wpb;
    if (g->linear) {
        const long blocks = ((long)(rows + rpw - 1) / rpw + wpb - 1) / wpb;
        g->blocks_per_xcd = (int)((blocks + 7) / 8);
    } else {
        const int waves = (g->stripe + rpw - 1) / rpw;
        g->blocks_per_xcd = (waves + wpb - 1) / wpb;
    }
    return true;
}

int matvec_compute_blocks(int rows, int n, int pro, int epi) {
    MatvecGeom g;
    return matvec_geometry(rows, n, pro, epi, &g) ? 8 * g.blocks_per_xcd : 0;
}

int matvec_block_threads(int rows, int n, int pro, int epi) {
    MatvecGeom g;
    return matvec_geometry(rows, n, pro, epi, &g) ? 64 * g.wpb : 0;
}

PrefetchDesc prefetch_for(const float *W, long ld, int rows, int n, int pro, int epi, int first_block,
                          int producer_threads, float *sink) {
    PrefetchDesc pf = {};
    MatvecGeom g;
    if (!W || ld % 4 || !matvec_geometry(rows, n, pro, epi, &g)) return pf;
    pf.base = W; pf.row_floats = ld; pf.rows = rows; pf.stripe = g.stripe;
    // 256 bytes per prefetch thread (two rounds of eight 16-byte loads);
    // prefetch blocks run with the producer kernel's block size.
    const long bytes_per_block = 256L * producer_threads;
    const long bytes_per_xcd = (long)g.stripe * ld * 4;
    const int per_xcd = (int)std::max<long>(1, std::min<long>(256, (bytes_per_xcd + bytes_per_block - 1) / bytes_per_block));
    pf.blocks = 8 * per_xcd;
    pf.first_block = first_block;
    pf.sink = sink;
    return pf;
}

// Host-side launcher: validates shapes and picks the kernel.
int launch_matvec(MatvecParams p, hipStream_t s, hipEvent_t e0, hipEvent_t e1, bool x_reread) {
    if (p.rows <= 0 || p.n <= 0) return set_error(PTMI_ERR_ARG, "matvec: rows=%d n=%d", p.rows, p.n);
    if (!p.W || !p.x || !p.y) return set_error(PTMI_ERR_ARG, "matvec: null pointer");
    if (p.ld < p.n) return set_error(PTMI_ERR_ARG, "matvec: ld=%ld < n=%d", p.ld, p.n);
    if (p.pro == PRO_ATTN_COMBINE &&
        (!p.att_o || !p.att_ml || !p.pos || p.att_heads <= 0 || p.att_heads > kMaxCombineHeads ||
         p.n % p.att_heads || p.n > kMaxCombineDim || p.att_chunk <= 0 || p.att_chunks <= 0 ||
         p.att_chunks > kMaxAttnChunks))
        return set_error(PTMI_ERR_ARG, "matvec: bad attention-combine description");
    const bool norm = p.pro == PRO_RMSNORM || p.pro == PRO_EMBED_RMSNORM;
    if (norm && !p.norm_w) return set_error(PTMI_ERR_ARG, "matvec: RMSNorm prologue without weights");
    if (p.pro == PRO_EMBED_RMSNORM && (!p.token || !p.x_out))
        return set_error(PTMI_ERR_ARG, "matvec: embedding prologue without token/x_out");
    const bool vec_ok = (p.n % 4 == 0) && (p.ld % 4 == 0) && aligned16(p.W) && aligned16(p.x) &&
                        (!norm || aligned16(p.norm_w)) &&
                        (p.pro != PRO_EMBED_RMSNORM || aligned16(p.x_out));
    const bool fused = p.pro != PRO_NONE || p.epi == EPI_QKV_ROPE || p.epi == EPI_SWIGLU;
    if (p.epi == EPI_QKV_ROPE &&
        ((p.q_rows & 1) || (p.kv_rows & 1) || p.head_dim <= 0 || !p.pos || !p.k_cache || !p.v_cache))
        return set_error(PTMI_ERR_ARG, "matvec: bad QKV epilogue description");
    if (p.epi == EPI_SWIGLU && (p.rows & 1))
        return set_error(PTMI_ERR_ARG, "matvec: SwiGLU needs an even row count");

    KernelFn fn = nullptr;
    int rpp = 1;
    MatvecGeom geo;
    if (x_reread && (p.pro != PRO_NONE || p.epi != EPI_STORE || p.pf.blocks))
        return set_error(PTMI_ERR_ARG, "matvec: the x re-read variant is a plain y = Wx");
    if (vec_ok && matvec_geometry(p.rows, p.n, p.pro, p.epi, &geo)) {
        if (x_reread) {
            switch (geo.lpr) {
            case 8: fn = pick_xr<8>(geo.it, geo.np); break;
            case 16: fn = pick_xr<16>(geo.it, geo.np); break;
            case 32: fn = pick_xr<32>(geo.it, geo.np); break;
            default: fn = pick_xr<64>(geo.it, geo.np); break;
            }
        } else {
            switch (geo.lpr) {
            case 8: fn = pick<8>(geo.it, geo.np, p.pro, p.epi); break;
            case 16: fn = pick<16>(geo.it, geo.np, p.pro, p.epi); break;
            case 32: fn = pick<32>(geo.it, geo.np, p.pro, p.epi); break;
            default: fn = pick<64>(geo.it, geo.np, p.pro, p.epi); break;
            }
        }
        if (!fn) return set_error(PTMI_ERR_ARG, "matvec: unsupported prologue/epilogue pair %d/%d", p.pro, p.epi);
        p.stripe = geo.stripe;
        p.rows_per_wave = geo.rows_per_wave;
        p.blocks_per_xcd = geo.blocks_per_xcd;
        p.linear = geo.linear;
        const int compute_blocks = 8 * geo.blocks_per_xcd;
        if (p.pf.blocks && p.pf.first_block != compute_blocks)
            return set_error(PTMI_ERR_ARG, "matvec: prefetch descriptor built for another grid");
        launch_k(fn, dim3((unsigned)(compute_blocks + p.pf.blocks)), dim3(geo.wpb * 64), 0, s, e0, e1, p);
        PTMI_HIP(hipGetLastError());
        return PTMI_OK;
    } else if (x_reread) {
        return set_error(PTMI_ERR_ARG, "matvec: the x re-read variant needs 16-byte rows of n <= %d", 64 * 9 * 4);
    } else if (vec_ok) {
        if (p.pf.blocks) return set_error(PTMI_ERR_ARG, "matvec: prefetch needs the register-resident kernel");
        if (p.pro != PRO_NONE || p.epi != EPI_STORE)
            return set_error(PTMI_ERR_ARG, "matvec: fused variants need n <= %d", 64 * 9 * 4);
        fn = k_matvec_long;
        rpp = 1;
    } else {
        if (fused) return set_error(PTMI_ERR_ARG, "matvec: fused variants need 16-byte aligned rows, n%%4==0");
        p.rows_per_wave = 1;
        const int blocks = (p.rows + kWaves - 1) / kWaves;
        launch_k(k_matvec_scalar, dim3(blocks), dim3(kWaves * 64), 0, s, e0, e1, p);
        PTMI_HIP(hipGetLastError());
        return PTMI_OK;
    }
    // rows per wave: a multiple of 2*rpp (row pairs for the fused epilogues),
    // at most 64, chosen for ~2048 waves in flight.
    const int step = 2 * rpp;
    const long target_waves = 2048;
    long rpw = (p.rows + target_waves - 1) / target_waves;
    rpw = ((rpw + step - 1) / step) * step;
    rpw = std::max<long>(rpw, step);
    rpw = std::min<long>(rpw, kMaxRowsPerWave);
    p.rows_per_wave = (int)rpw;
    const long waves = (p.rows + rpw - 1) / rpw;
    const long blocks = (waves + kWaves - 1) / kWaves;
    launch_k(fn, dim3((unsigned)blocks), dim3(kWaves * 64), 0, s, e0, e1, p);
    PTMI_HIP(hipGetLastError());
    return PTMI_OK;
}

}  // namespace ptmi
