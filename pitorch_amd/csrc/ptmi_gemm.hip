// fp32 GEMMs on the CDNA4 matrix cores: C[M,N] (+)= op(A)[M,K] . op(B)[K,N]
// with v_mfma_f32_16x16x4_f32.  These replace the training backward's
// per-position matvecs / CPU outer products:
//   dW = dY^T X  (TN) — matmul_backward_weight_batched, pt_train.c:475-492
//   dX = dY W    (NN) — backward_input_pretrans, pt_train.c:442-453
//   Y  = X W^T   (NT) — the batched form of the training forward's matvecs
//
// Block tile TMxTN (64x64, or 32x32 for small output grids), K step 32,
// 256 threads = 4 waves in a 2x2 grid, each wave a (TM/2)x(TN/2) sub-tile
// of 16x16 MFMA blocks.  Tiles are staged in LDS k-major (As[k][m],
// Bs[k][n], columns XOR-swizzled so no LDS access has bank conflicts).  Two K
// tiles are in flight in registers while a third feeds the matrix cores
// from LDS (double-buffered), so each tile's global latency is covered by
// two K steps of MFMAs.  Operand layout of the 16x16x4 f32 MFMA (CDNA3/4):
// lane l supplies A[l%16][l/16] and B[l/16][l%16]; result register r of lane
// l is C[4*(l/16)+r][l%16].
// Long-K GEMMs with small output grids split K over blockIdx.z into a
// workspace and reduce in split order afterwards (deterministic, no
// atomics).
#include "ptmi_internal.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <utility>

namespace ptmi {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BK = 32;
constexpr int kXcdGrid = 768;             // grids this large take their tiles in XCD order
constexpr int kRing64 = 2, kRing32 = 2;   // K tiles in flight per block tile size

struct GemmArgs {
    const float *A; long lda;
    const float *B; long ldb;
    float *C; long ldc;
    const float *Cin;      // accumulate: C = Cin + op(A).op(B) (Cin == C in place), same ldc
    int M, N, K;
    int accumulate;
    float *partial;        // split-K workspace [splits][M][N] or null
    int k_per_split;
    GemmEpi epi;           // fused element-wise epilogue (whole-K launches only)
    GemmNorm nrm;          // fused RMSNorm of the A rows (NT, whole K)
    float *upd;            // fused SGD step of the weight C is the gradient of (TnGemm), or null
    const float *lr;
    const unsigned *keep;
};

// One GEMM of a grouped launch: its arguments and its range of tiles.
struct GemmGroupDesc {
    GemmArgs g;
    int tiles_n;           // tiles along N
    int tile0;             // first block of this GEMM in the grouped grid
};

// Read by loads whose element lies outside the operand (ragged edges and
// the K tail), so every load is unconditional and needs no select after it.
__device__ __align__(16) float g_gemm_zero[16] = {};

// One operand tile (R rows of the M or N side x 32 k) per K step; each of
// the 256 threads moves E = R*32/256 floats (8 or 4).  KMAJOR: the operand
// is stored with k as the row index (A^T for TN, B for NN/TN); otherwise k
// is the contiguous index.
//   KMAJOR:  thread -> (k = tid/(R/E),     idx = E*(tid%(R/E)) + c)
//   !KMAJOR: thread -> (idx = tid/(32/E),  k = E*(tid%(32/E)) + c)
// VEC: 16-byte float4 loads; the launcher guarantees aligned rows and a
// contiguous extent (idx_lim for KMAJOR, K otherwise) that is a multiple of
// 4, so a float4 is either wholly inside the operand or wholly outside.
// Elements outside read g_gemm_zero: only the address is selected, before
// the load, so the loads of a tile stay in flight together (a select on the
// loaded value, or a branch, makes the compiler wait for every load issued
// so far).
template <bool KMAJOR, int R, bool VEC>
__device__ __forceinline__ void load_tile(const float *P, long ld, int idx_lim, int i0, int k0, int kend, int tid,
                                          float (&r)[R * BK / 256]) {
    constexpr int E = R * BK / 256;
    const float *zero = g_gemm_zero;
    if (KMAJOR) {
        const int k = k0 + tid / (R / E), i = i0 + E * (tid % (R / E));
        const bool kin = k < kend;
        const float *row = P + (long)(kin ? k : 0) * ld;
        if constexpr (VEC) {
#pragma unroll
            for (int c = 0; c < E; c += 4) {
                const bool in = kin && i + c < idx_lim;
                const float4 v = *reinterpret_cast<const float4 *>(in ? row + i + c : zero + c);
                r[c] = v.x; r[c + 1] = v.y; r[c + 2] = v.z; r[c + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int c = 0; c < E; c++) r[c] = *((kin && i + c < idx_lim) ? row + i + c : zero + c);
        }
    } else {
        const int i = i0 + tid / (BK / E), k = k0 + E * (tid % (BK / E));
        const bool iin = i < idx_lim;
        const float *row = P + (long)(iin ? i : 0) * ld;
        if constexpr (VEC) {
#pragma unroll
            for (int c = 0; c < E; c += 4) {
                const bool in = iin && k + c < kend;
                const float4 v = *reinterpret_cast<const float4 *>(in ? row + k + c : zero + c);
                r[c] = v.x; r[c + 1] = v.y; r[c + 2] = v.z; r[c + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int c = 0; c < E; c++) r[c] = *((iin && k + c < kend) ? row + k + c : zero + c);
        }
    }
}

// LDS holds each operand tile k-major, S[k][col] with rows of R floats, the
// column XOR-swizzled by row (and, for 64-wide k-major tiles, by column
// half) so that, with LDS's 32 banks and a wave64 b32 access served as two
// half-waves (b128 as four 8-lane groups), every access below is
// conflict-free:
//  * the MFMA operand reads (a half-wave reads rows k, k+1 at 16 columns):
//    bit 4 of the swizzle differs between rows k and k+1;
//  * the transposing b32 stores of !KMAJOR operands (a half-wave writes one
//    row per k group at 8 or 4 consecutive columns): the swizzle's bits
//    3..4 (R = 64) or 2..4 (R = 32) take a different value per k group;
//  * the b128 stores of KMAJOR operands (8 lanes write one row, 4 floats
//    each, at a stride of E floats): for R = 64 the upper column half
//    moves by 4 banks.
// Bits 0..1 are never swizzled, so float4 chunks stay whole.
template <bool KMAJOR, int R>
__device__ __forceinline__ int lds_col(int r, int c) {
    if constexpr (KMAJOR) {
        if constexpr (R == 64) return c ^ ((r & 1) << 4) ^ (((c >> 5) & 1) << 2);
        return c ^ ((r & 1) << 4);
    } else if constexpr (R == 64) {
        return c ^ ((((r & 1) ^ ((r >> 3) & 1)) << 4) | (((r >> 4) & 1) << 3));
    } else {
        return c ^ ((((r & 1) ^ ((r >> 2) & 1)) << 4) | (((r >> 3) & 1) << 3) | (((r >> 4) & 1) << 2));
    }
}

template <bool KMAJOR, int R>
__device__ __forceinline__ void store_tile(float (*S)[R], int tid, const float (&r)[R * BK / 256]) {
    constexpr int E = R * BK / 256;
    if (KMAJOR) {
        const int k = tid / (R / E), i = E * (tid % (R / E));
#pragma unroll
        for (int c = 0; c < E; c += 4)
            *reinterpret_cast<float4 *>(&S[k][lds_col<KMAJOR, R>(k, i + c)]) =
                make_float4(r[c], r[c + 1], r[c + 2], r[c + 3]);
    } else {
        const int i = tid / (BK / E), k = E * (tid % (BK / E));
#pragma unroll
        for (int c = 0; c < E; c++) S[k + c][lds_col<KMAJOR, R>(k + c, i)] = r[c];
    }
}

// Epilogue of one wave's FM x FN 16x16 blocks: block (i, j) of the wave
// covers rows mb + 16i .. and columns nb + 16j ..; lane l holds rows
// 4*(l/16) + r, column l%16 of it (the 16x16x4 MFMA result layout).
template <int EPI, int FM, int FN>
__device__ __forceinline__ void gemm_store(const GemmArgs &g, const floatx4 (&acc)[FM][FN], int mb, int nb, int z,
                                           int li, int lk, const float *rs = nullptr, int rs_m0 = 0) {
    const float lrv = g.upd ? *g.lr : 0.0f;
    // C[4*(l/16)+r][l%16] of each 16x16 block; columns n and n^1 of a row sit
    // in lanes l and l^1, which the fused epilogues pair with a DPP swap
    // (every lane reaches it: bounds are checked after).
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = nb + j * 16 + li;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mb + i * 16 + 4 * lk + r;
                float v = acc[i][j][r];
                if (rs) v *= rs[m - rs_m0];                     // fused RMSNorm: the row's 1/rms
                if constexpr (EPI == GEMM_EPI_ROPE) {
                    // RoPE of the q and k columns at position m (pt_ops.c:33-49;
                    // training forward pt_train.c:217)
                    const float pv = dpp_xor1(v);
                    if (n < 2 * g.epi.rope_dim) {
                        const int ip = (n < g.epi.rope_dim ? n : n - g.epi.rope_dim) & ~1;
                        float c, sn;
                        d_rope_cs(ip, g.epi.head_dim, m, &c, &sn);
                        v = (n & 1) ? pv * sn + v * c : v * c - pv * sn;
                    }
                } else if constexpr (EPI == GEMM_EPI_SWIGLU) {
                    // columns (2i, 2i+1) = (h1, h3): out[m][i] = (h1*sigmoid(h1))*h3,
                    // the training form of silu (pt_train.c:280-284)
                    const float pv = dpp_xor1(v);
                    if (!(n & 1) && n < g.N && m < g.M) {
                        const float sig = 1.0f / (1.0f + d_expf(-v));
                        g.epi.out[(long)m * g.epi.ld + (n >> 1)] = (v * sig) * pv;
                    }
                }
                if constexpr (EPI == GEMM_EPI_SWIGLU_BWD) {
                    // silu*gate backward (pt_train.c:696-721) into the interleaved
                    // (d_h1, d_h3) columns, plus silu(h1)*h3 for dW2
                    if (n < g.N && m < g.M) {
                        const float *hp = g.epi.aux + (long)m * g.epi.aux_ld + 2 * n;
                        const float h1 = hp[0], h3 = hp[1];
                        const float sig = 1.0f / (1.0f + d_expf(-h1));
                        const float silu_val = h1 * sig;
                        g.epi.out2[(long)m * g.epi.ld2 + n] = silu_val * h3;
                        const float d_silu = v * h3;
                        float *dp = g.epi.out + (long)m * g.epi.ld + 2 * n;
                        dp[1] = v * silu_val;
                        dp[0] = d_silu * sig * (1.0f + h1 * (1.0f - sig));
                    }
                    continue;                                   // d_sh itself is not kept
                }
                if (n >= g.N || m >= g.M) continue;
                if (g.partial) {
                    g.partial[((long)z * g.M + m) * g.N + n] = v;
                } else {
                    const long o = (long)m * g.ldc + n;
                    const float cv = g.accumulate ? g.Cin[o] + v : v;
                    g.C[o] = cv;
                    // sgd_step (pt_train.c:870-873) on the weight this gradient belongs to
                    if (g.upd && !(g.keep && ((g.keep[m >> 5] >> (m & 31)) & 1u))) g.upd[o] -= lrv * cv;
                }
            }
        }
    }
}

// Fused RMSNorm: the block of N tile j stores its share of rows m0 ..
// m0+R-1 (float4 columns [j*c4, (j+1)*c4) of K/4, c4 = ceil(K/4 / tiles))
// of X (to x_out when completed here) and of X * inv * w (to xn_out), all
// loads of a pass in flight together; the block of tile 0 also marks the
// rows' tokens (EMBED, rows < M-1) in tok_bits.
template <int NORM, int R>
__device__ __forceinline__ void norm_rows_out(const GemmArgs &g, int m0, int j, int tiles, const float *inv) {
    const GemmNorm &nm = g.nrm;
    const int K4 = g.K / 4, c4 = (K4 + tiles - 1) / tiles, c_lo = j * c4, c_n = min(c4, K4 - c_lo);
    const int tid = threadIdx.x;
    const float *zero = g_gemm_zero;
    for (int e = tid; e < R * c_n; e += 256) {
        const int r = e / c_n, m = m0 + r;
        const bool in = m < g.M;
        const long col = 4L * (c_lo + (e - r * c_n));
        const long o = (long)min(m, g.M - 1) * g.K + col;
        float4 x;
        if constexpr (NORM == GEMM_NORM_SPLITS) {
            float4 p[kNormSplits];
#pragma unroll
            for (int zz = 0; zz < kNormSplits; zz++)
                p[zz] = *reinterpret_cast<const float4 *>(zz < nm.pk.splits ? nm.pk.parts + zz * nm.pk.stride + o : zero);
            const float4 c = *reinterpret_cast<const float4 *>(nm.cin ? nm.cin + o : zero);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int zz = 0; zz < kNormSplits; zz++) {
                const bool use = zz < nm.pk.splits;
                v.x = use ? v.x + p[zz].x : v.x;
                v.y = use ? v.y + p[zz].y : v.y;
                v.z = use ? v.z + p[zz].z : v.z;
                v.w = use ? v.w + p[zz].w : v.w;
            }
            x = nm.cin ? make_float4(c.x + v.x, c.y + v.y, c.z + v.z, c.w + v.w) : v;
        } else if constexpr (NORM == GEMM_NORM_EMBED) {
            x = *reinterpret_cast<const float4 *>(nm.emb + (long)nm.tok[min(m, g.M - 1)] * g.K + col);
        } else {
            x = *reinterpret_cast<const float4 *>(g.A + o);
        }
        const float4 w = *reinterpret_cast<const float4 *>(nm.w + col);
        if (!in) continue;
        if constexpr (NORM != GEMM_NORM_PLAIN) *reinterpret_cast<float4 *>(nm.x_out + o) = x;
        const float iv = inv[r];
        *reinterpret_cast<float4 *>(nm.xn_out + o) = make_float4(x.x * iv * w.x, x.y * iv * w.y, x.z * iv * w.z, x.w * iv * w.w);
    }
    if constexpr (NORM == GEMM_NORM_EMBED) {
        const int m = m0 + tid;
        if (j == 0 && tid < R && m < g.M - 1) {
            const int tk = nm.tok[m];
            atomicOr(&nm.tok_bits[tk >> 5], 1u << (tk & 31));
        }
    }
}

// One TMxTN output tile of g at (m0, n0) over K range split z.  The LDS
// tiles use the swizzled layout of lds_col.
template <bool AT, bool BT, int TM, int TN, int P, bool VEC, int EPI = GEMM_EPI_NONE, int NORM = 0>
__device__ __forceinline__ void gemm_tile(const GemmArgs &g, int m0, int n0, int z) {
    constexpr int FM = TM / 32, FN = TN / 32;          // 16x16 MFMA blocks per wave
    constexpr int EA = TM * BK / 256, EB = TN * BK / 256;
    static_assert(NORM == 0 || (!AT && TM == 32 && VEC && EA == 4), "fused norm: NT, 32-row float4 A tiles");
    __shared__ float As[2][BK][TM];
    __shared__ float Bs[2][BK][TN];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 15, lk = lane >> 4;
    const int kb = z * g.k_per_split;
    const int kend = min(g.K, kb + g.k_per_split);
    const int nk = kb < kend ? (kend - kb + BK - 1) / BK : 0;

    floatx4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // P K tiles in flight in a register ring (tile t in slot t % P); the
    // loop is unrolled by P so every slot index is a compile-time constant.
    float ra[P][EA], rb[P][EB];
    // Fused RMSNorm: thread tid owns A row na_i and k offset na_k of every K
    // step (the load_tile mapping); the ring holds the raw row values (the
    // split-K partials and the addend, summed at the LDS store) and the norm
    // weights; the A tile takes x * w, and the row's sum of squares builds up.
    constexpr int NL = NORM == GEMM_NORM_SPLITS ? kNormSplits + 1 : 1;
    const int na_i = m0 + tid / (BK / EA), na_k = EA * (tid % (BK / EA));
    float4 nr[P][NL], ng[P];
    float nss = 0.0f;
    const float *na_row = g.A + (long)min(na_i, g.M - 1) * g.lda;
    if constexpr (NORM == GEMM_NORM_EMBED) na_row = g.nrm.emb + (long)g.nrm.tok[min(na_i, g.M - 1)] * g.K;
    auto load = [&](int s, int slot, float (&xa)[EA], float (&xb)[EB]) {
        if constexpr (NORM != 0) {
            const float *zero = g_gemm_zero;
            const int k = kb + s * BK + na_k;
            const bool in = na_i < g.M && k < kend;
            if constexpr (NORM == GEMM_NORM_SPLITS) {
                const long o = (long)min(na_i, g.M - 1) * g.K + k;
#pragma unroll
                for (int zz = 0; zz < kNormSplits; zz++)
                    nr[slot][zz] = *reinterpret_cast<const float4 *>(
                        in && zz < g.nrm.pk.splits ? g.nrm.pk.parts + zz * g.nrm.pk.stride + o : zero);
                nr[slot][kNormSplits] = *reinterpret_cast<const float4 *>(in && g.nrm.cin ? g.nrm.cin + o : zero);
            } else {
                nr[slot][0] = *reinterpret_cast<const float4 *>(in ? na_row + k : zero);
            }
            ng[slot] = *reinterpret_cast<const float4 *>(in ? g.nrm.w + k : zero);
        } else {
            load_tile<AT, TM, VEC>(g.A, g.lda, g.M, m0, kb + s * BK, kend, tid, xa);
        }
        load_tile<!BT, TN, VEC>(g.B, g.ldb, g.N, n0, kb + s * BK, kend, tid, xb);
    };
    auto store = [&](int s, int slot, const float (&xa)[EA], const float (&xb)[EB]) {
        if constexpr (NORM != 0) {
            float4 x = nr[slot][0];
            if constexpr (NORM == GEMM_NORM_SPLITS) {
                // the standalone kernel's order: ((0 + p0) + p1) + ..., then cin + sum
                float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int zz = 0; zz < kNormSplits; zz++) {
                    const bool use = zz < g.nrm.pk.splits;
                    v.x = use ? v.x + nr[slot][zz].x : v.x;
                    v.y = use ? v.y + nr[slot][zz].y : v.y;
                    v.z = use ? v.z + nr[slot][zz].z : v.z;
                    v.w = use ? v.w + nr[slot][zz].w : v.w;
                }
                const float4 c = nr[slot][kNormSplits];
                x = g.nrm.cin ? make_float4(c.x + v.x, c.y + v.y, c.z + v.z, c.w + v.w) : v;
            }
            nss += x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
            const float4 w = ng[slot];
            const float xw[EA] = {x.x * w.x, x.y * w.y, x.z * w.z, x.w * w.w};
            store_tile<AT, TM>(As[s & 1], tid, xw);
        } else {
            store_tile<AT, TM>(As[s & 1], tid, xa);
        }
        store_tile<!BT, TN>(Bs[s & 1], tid, xb);
    };
    // The operands of k group kk+4*RA are read from LDS before the MFMAs of
    // group kk issue, so their latency overlaps RA groups of MFMAs (RA = 2
    // and 3 measured no faster).
    constexpr int RA = 1;
    auto compute = [&](int s) {
        const int buf = s & 1;
        float a[RA + 1][FM], b[RA + 1][FN];
        auto read = [&](int kk, float (&ar)[FM], float (&br)[FN]) {
#pragma unroll
            for (int i = 0; i < FM; i++) ar[i] = As[buf][kk + lk][lds_col<AT, TM>(kk + lk, wm * (TM / 2) + i * 16 + li)];
#pragma unroll
            for (int j = 0; j < FN; j++) br[j] = Bs[buf][kk + lk][lds_col<!BT, TN>(kk + lk, wn * (TN / 2) + j * 16 + li)];
        };
#pragma unroll
        for (int r = 0; r < RA; r++) read(4 * r, a[r], b[r]);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            const int c = (kk / 4) % (RA + 1);
            if (kk + 4 * RA < BK) read(kk + 4 * RA, a[(kk / 4 + RA) % (RA + 1)], b[(kk / 4 + RA) % (RA + 1)]);
            __builtin_amdgcn_sched_barrier(0);              // keep the reads ahead of the MFMAs
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c][i], b[c][j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

#pragma unroll
    // Loads are unconditional (tiles past the K range read zeros): a load
    // under a branch leaves the compiler unsure how many loads are in flight,
    // and it then waits for all of them, which empties the ring.
    for (int t = 0; t < P; t++) load(t, t, ra[t], rb[t]);
    store(0, 0, ra[0], rb[0]);
    __syncthreads();
    // Step s: tile s is in LDS; its register slot (s % P) is free, so tile
    // s+P is fetched into it; tile s+1 goes to the other LDS buffer.  Full
    // groups of P steps run without branches; the last nk % P steps follow.
    int s0 = 0;
    for (; s0 + P <= nk; s0 += P) {
#pragma unroll
        for (int u = 0; u < P; u++) {
            load(s0 + u + P, u, ra[u], rb[u]);
            __builtin_amdgcn_sched_barrier(0);              // issue the loads before the MFMAs
            compute(s0 + u);
            store(s0 + u + 1, (u + 1) % P, ra[(u + 1) % P], rb[(u + 1) % P]);
            __syncthreads();
        }
    }
#pragma unroll
    for (int u = 0; u + 1 < P; u++) {
        if (s0 + u < nk) {                                  // uniform
            compute(s0 + u);
            store(s0 + u + 1, (u + 1) % P, ra[(u + 1) % P], rb[(u + 1) % P]);
            __syncthreads();
        }
    }

    if constexpr (NORM != 0) {
        // 1/rms of the block's rows (the standalone kernel's formula); every
        // N tile's block stores its share of the rows and normalized rows
        __shared__ float n_inv[TM];
        nss = group_sum<BK / EA>(nss);
        if (tid % (BK / EA) == 0) n_inv[tid / (BK / EA)] = 1.0f / d_sqrtf(nss / (float)g.K + 1e-5f);
        __syncthreads();
        norm_rows_out<NORM, TM>(g, m0, n0 / TN, (g.N + TN - 1) / TN, n_inv);
        gemm_store<EPI, FM, FN>(g, acc, m0 + wm * (TM / 2), n0 + wn * (TN / 2), z, li, lk, n_inv, m0);
    } else {
        gemm_store<EPI, FM, FN>(g, acc, m0 + wm * (TM / 2), n0 + wn * (TN / 2), z, li, lk);
    }
}

// ── Direct-to-LDS tiles for the large training GEMMs ─────────────────────
// gfx950's global_load_lds_dwordx4 moves a 16-byte chunk per lane from
// global memory straight into LDS, at the wave's LDS base + 16*lane (lane
// layout checked on the MI355X).  No staging registers and no LDS store
// instructions, so 128- and 256-row tiles fit with two waves per SIMD.
// Each operand tile keeps its global layout in LDS, permuted in whole
// 16-byte chunks (the only granularity a DMA load can place):
//  * k-contiguous operands ([i][k]: A of NN/NT, B^T of NT): rows of BK=32
//    floats (128 bytes), chunk c of row i at slot c ^ kc_swz(i).  A lane
//    reads the 4 k of its row for 4 MFMA steps as one b128 (lane group g
//    takes k = 4g..4g+3 of each 16-k group).  A b128 read serves 16 lanes
//    (16 rows) at a time across the 64 banks, where rows i and i+8 start on
//    the same bank; kc_swz gives the 16 rows 16 distinct bank groups.  With
//    c ^ (i & 7) alone the 32x32x2 NT tile measured 45.5% LDS conflict
//    cycles (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE), with kc_swz 7.7%
//    (one cycle per 64-lane b32 write of its store staging), at the same
//    speed and bits;
//  * k-major operands ([k][i]: A^T of TN, B of NN/TN): rows of TI floats,
//    the column XOR-ed with 16 in rows whose bit 2 of k is set; the two k
//    rows a half-wave reads (g = 0, 1) then sit 16 banks apart.
// Both operands use the same order of k inside a 16-k group (lane group g,
// step s -> k = 4g + s), so every product pairs the same k.
// Two LDS stages: the loads of tile s+1 are issued before the MFMAs of tile
// s and waited for (vmcnt, in order) at the next step's barrier.
// The classifier's weight gradient (TN) runs on these tiles, its forward
// (NT) on the 32x32x2 form below (gemm_tile_dl32).
// Measured on the MI355X against the register-ring kernel (launches back to
// back, same inputs, same bits): NT 256x32000x288 with 256x128 tiles, 47.2
// vs 51.3 us; TN 32000x288x255 with 64x96 tiles, 55.5 vs 58.7 us, and with
// 128x96 tiles on 8 waves (4x2) 51.1-52.9 vs 53.6-55.1 us (graph-replayed,
// same output bits; 128x96 on 4 or 8x1 waves, 256x96, 64x96 on 8 waves,
// 64x288 and 128x288 were slower).  NT 256x128 on 8x1 or 2x4 waves and
// 256x64 tiles were no faster than 4x2.  Deeper
// stage rings, 64-k stages, and loads interleaved one per MFMA k step were
// all slower; so were these tiles on the per-layer shapes (5-16 us against
// 5-10 us) and on the long-K NN (split K, 68 vs 60 us).
constexpr int kDlStages = 2;

// Chunk-slot swizzle of row i of a k-contiguous tile: i & 7 spreads 8
// consecutive rows over the 8 slots; bit 3 of i moves rows i and i+8 to
// different slots.
__device__ __forceinline__ int kc_swz(int i) { return (i & 7) ^ ((i >> 3) & 1); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {                   // s_waitcnt vmcnt(N), other counters untouched
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// This thread's DMA loads of one operand tile (TI rows of the M or N side x
// BK k, k0 = first k) into `lds`; 64-chunk regions are dealt to the NW
// waves round-robin, and a wave with no region left loads zeros into `junk`
// so that every wave issues the same number of loads.
template <bool KMAJOR, int TI, int NW>
__device__ __forceinline__ void dl_issue(const float *P, long ld, int ilim, int i0, int k0, int kend, float *lds,
                                         float *junk, int wave, int lane) {
    constexpr int CPI = BK / 4;                          // chunks per row, k-contiguous layout
    constexpr int R = TI * CPI / 64;
#pragma unroll
    for (int j = 0; j < (R + NW - 1) / NW; j++) {
        const int rgn = j * NW + wave;
        const bool real = rgn < R;                       // wave-uniform
        const int S = (real ? rgn : 0) * 64 + lane;      // chunk slot in the tile
        const float *src = g_gemm_zero;
        if constexpr (KMAJOR) {
            constexpr int CPR = TI / 4;                  // chunks per LDS row
            const int k = S / CPR, t = S % CPR;
            const int i = i0 + 4 * (t ^ (((k >> 2) & 1) << 2)), kk = k0 + k;
            if (real && kk < kend && i < ilim) src = P + (long)kk * ld + i;
        } else {
            const int i = S / CPI, t = S % CPI;
            const int ii = i0 + i, kk = k0 + 4 * (t ^ kc_swz(i));
            if (real && ii < ilim && kk < kend) src = P + (long)ii * ld + kk;
        }
        typedef const void __attribute__((address_space(1))) *gptr;
        typedef void __attribute__((address_space(3))) *lptr;
        __builtin_amdgcn_global_load_lds((gptr)src, (lptr)(real ? lds + rgn * 256 : junk), 16, 0, 0);
    }
}

// One TMxTN output tile on WM x WN waves (each (TM/WM) x (TN/WN)).
// AK: A stored [K][M] (TN); BKM: B stored [K][N] (NN, TN).
template <bool AK, bool BKM, int TM, int TN, int WM, int WN, int EPI = GEMM_EPI_NONE>
__device__ __forceinline__ void gemm_tile_dl(const GemmArgs &g, int m0, int n0, int z) {
    constexpr int NW = WM * WN, NS = kDlStages, CPI = BK / 4;
    constexpr int FM = TM / WM / 16, FN = TN / WN / 16;
    static_assert(FM * WM * 16 == TM && FN * WN * 16 == TN, "tile");
    constexpr int STAGE = (TM + TN) * BK;
    constexpr int LPT = (TM * CPI / 64 + NW - 1) / NW + (TN * CPI / 64 + NW - 1) / NW;
    static_assert((NS - 2) * LPT < 64, "vmcnt");
    __shared__ __align__(16) float smem[NS * STAGE + 256];
    float *junk = smem + NS * STAGE;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 15, lk = lane >> 4;
    const int kb = z * g.k_per_split;
    const int kend = min(g.K, kb + g.k_per_split);
    const int nk = kb < kend ? (kend - kb + BK - 1) / BK : 0;

    floatx4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto issue = [&](int t) {
        float *st = smem + (t % NS) * STAGE;
        const int k0 = kb + t * BK;
        dl_issue<AK, TM, NW>(g.A, g.lda, g.M, m0, k0, kend, st, junk, wave, lane);
        dl_issue<BKM, TN, NW>(g.B, g.ldb, g.N, n0, k0, kend, st + TM * BK, junk, wave, lane);
    };
    // MFMA operands of 16-k group q: lane group lk takes k = 16q + 4lk + s
    // in step s (a float4 per fragment, one k per component).
    auto read_a = [&](const float *st, int q, floatx4 (&a)[FM]) {
#pragma unroll
        for (int f = 0; f < FM; f++) {
            const int i = wm * (TM / WM) + f * 16 + li;
            if constexpr (AK) {
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const int k = 16 * q + 4 * lk + s;
                    a[f][s] = st[k * TM + (i ^ (((k >> 2) & 1) << 4))];
                }
            } else {
                a[f] = *reinterpret_cast<const floatx4 *>(st + (i * CPI + ((4 * q + lk) ^ kc_swz(i))) * 4);
            }
        }
    };
    auto read_b = [&](const float *st, int q, floatx4 (&b)[FN]) {
        const float *sb = st + TM * BK;
#pragma unroll
        for (int h = 0; h < FN; h++) {
            const int i = wn * (TN / WN) + h * 16 + li;
            if constexpr (BKM) {
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const int k = 16 * q + 4 * lk + s;
                    b[h][s] = sb[k * TN + (i ^ (((k >> 2) & 1) << 4))];
                }
            } else {
                b[h] = *reinterpret_cast<const floatx4 *>(sb + (i * CPI + ((4 * q + lk) ^ kc_swz(i))) * 4);
            }
        }
    };

    if (nk > 0) issue(0);
    for (int s = 0; s < nk; s++) {
        // tile s has landed in every wave's share once each wave's own
        // loads are done (vmcnt) and all waves passed the barrier; the
        // barrier also ends every read of the stage tile s+1 overwrites
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 1 < nk) issue(s + 1);
        const float *st = smem + (s % NS) * STAGE;
        floatx4 a[2][FM], b[2][FN];
        read_a(st, 0, a[0]);
        read_b(st, 0, b[0]);
        read_a(st, 1, a[1]);
        read_b(st, 1, b[1]);
#pragma unroll
        for (int q = 0; q < 2; q++)
#pragma unroll
            for (int ss = 0; ss < 4; ss++)
#pragma unroll
                for (int f = 0; f < FM; f++)
#pragma unroll
                    for (int h = 0; h < FN; h++)
                        acc[f][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q][f][ss], b[q][h][ss], acc[f][h], 0, 0, 0);
    }
    gemm_store<EPI, FM, FN>(g, acc, m0 + wm * (TM / WM), n0 + wn * (TN / WN), z, li, lk);
}

// f(integral_constant<int, s>) for s = S...
template <typename F, int... S>
__device__ __forceinline__ void unrolled(F &f, std::integer_sequence<int, S...>) {
    (f(std::integral_constant<int, S>{}), ...);
}

// The per-layer GEMMs' 32x32 tile with every K tile of its split in flight
// at once: the block issues the DMA loads of all NSK tiles (each into its
// own LDS stage; tiles past the split's K range load zeros) before its first
// MFMA, and starts tile s once the loads behind it are the only ones left
// (vmcnt counts them).  The register ring holds one or two tiles ahead, so
// each of its K steps waits about one load latency; here the block waits
// for about one.  Operand layout, MFMA k order and epilogue as
// gemm_tile_dl with 2 x 2 waves of 16 x 16.  NT (B^T k-contiguous) or NN
// (BKM: B stored [K][N]).
template <bool BKM, int NSK, int EPI>
__device__ __forceinline__ void gemm_tile_panel(const GemmArgs &g, int m0, int n0, int z) {
    constexpr int TM = 32, TN = 32, WN = 2, NW = 4, CPI = BK / 4;
    constexpr int STAGE = (TM + TN) * BK;
    constexpr int LPT = (TM * CPI / 64 + NW - 1) / NW + (TN * CPI / 64 + NW - 1) / NW;
    static_assert((NSK - 1) * LPT < 64, "vmcnt");
    __shared__ __align__(16) float smem[NSK * STAGE + 256];
    float *junk = smem + NSK * STAGE;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 15, lk = lane >> 4;
    const int kb = z * g.k_per_split;
    const int kend = min(g.K, kb + g.k_per_split);
    const int nk = kb < kend ? (kend - kb + BK - 1) / BK : 0;
#pragma unroll
    for (int t = 0; t < NSK; t++) {
        float *st = smem + t * STAGE;
        dl_issue<false, TM, NW>(g.A, g.lda, g.M, m0, kb + t * BK, kend, st, junk, wave, lane);
        dl_issue<BKM, TN, NW>(g.B, g.ldb, g.N, n0, kb + t * BK, kend, st + TM * BK, junk, wave, lane);
    }
    floatx4 acc[1][1] = {{floatx4{0.f, 0.f, 0.f, 0.f}}};
    const int ia = wm * 16 + li, ib = wn * 16 + li;
    // step s, unrolled (each wait takes a constant count)
    auto step = [&](auto sc) {
        constexpr int s = decltype(sc)::value;
        wait_vmcnt<(NSK - 1 - s) * LPT>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s < nk) {                                               // uniform
            const float *st = smem + s * STAGE, *sb = st + TM * BK;
            floatx4 a[2], b[2];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                a[q] = *reinterpret_cast<const floatx4 *>(st + (ia * CPI + ((4 * q + lk) ^ kc_swz(ia))) * 4);
                if constexpr (BKM) {
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int k = 16 * q + 4 * lk + u;
                        b[q][u] = sb[k * TN + (ib ^ (((k >> 2) & 1) << 4))];
                    }
                } else {
                    b[q] = *reinterpret_cast<const floatx4 *>(sb + (ib * CPI + ((4 * q + lk) ^ kc_swz(ib))) * 4);
                }
            }
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int u = 0; u < 4; u++)
                    acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q][u], b[q][u], acc[0][0], 0, 0, 0);
        }
    };
    unrolled(step, std::make_integer_sequence<int, NSK>{});
    gemm_store<EPI, 1, 1>(g, acc, m0 + wm * 16, n0 + wn * 16, z, li, lk);
}

// The NT direct-to-LDS tile on v_mfma_f32_32x32x2_f32 (the classifier's
// forward: both operands k-contiguous, same LDS layout and DMA loads as
// gemm_tile_dl).  In 8-k block q, lane half h = l/32 of a 32-lane group
// reads chunk 2q + h of its row as one b128, so step s pairs k = 8q + s
// (h = 0) with k = 8q + 4 + s (h = 1); A and B use the same order.  The 8
// lanes of a b128 access phase hit 8 distinct chunk slots, as in
// gemm_tile_dl.  C[(v/4)*8 + 4h + v%4][l%32] is component v of the lane's
// 16 sums; the tile goes out through LDS as whole rows, a float4 per lane.
// Measured on the MI355X for the 15M classifier (256 x 32000 x 288,
// interleaved launches): 44.5-49.9 us against 45.7-51.4 us for the 16x16x4
// tile, the same bits on integer-valued operands.  Four waves per SIMD
// (16-wave 256x128 tiles, or two 128x128 workgroups per CU) and a third LDS
// stage gave no further gain: each 32-k step costs ~4.0 us in every form,
// the rate of one wave's MFMA issue.
typedef float floatx16 __attribute__((ext_vector_type(16)));
template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void gemm_tile_dl32(const GemmArgs &g, int m0, int n0, int z) {
    constexpr int NW = WM * WN, NS = kDlStages, CPI = BK / 4;
    constexpr int FM = TM / WM / 32, FN = TN / WN / 32;
    static_assert(FM * WM * 32 == TM && FN * WN * 32 == TN, "tile");
    constexpr int STAGE = (TM + TN) * BK;
    __shared__ __align__(16) float smem[NS * STAGE + 256];
    float *junk = smem + NS * STAGE;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 31, lh = lane >> 5;
    const int kb = z * g.k_per_split;
    const int kend = min(g.K, kb + g.k_per_split);
    const int nk = kb < kend ? (kend - kb + BK - 1) / BK : 0;

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.0f;

    auto issue = [&](int t) {
        float *st = smem + (t % NS) * STAGE;
        const int k0 = kb + t * BK;
        dl_issue<false, TM, NW>(g.A, g.lda, g.M, m0, k0, kend, st, junk, wave, lane);
        dl_issue<false, TN, NW>(g.B, g.ldb, g.N, n0, k0, kend, st + TM * BK, junk, wave, lane);
    };
    // row i of a k-contiguous tile, k = 8q + 4h + s in component s
    auto rd = [&](const float *base, int i, int q) {
        return *reinterpret_cast<const floatx4 *>(base + (i * CPI + ((2 * q + lh) ^ kc_swz(i))) * 4);
    };

    if (nk > 0) issue(0);
    for (int s = 0; s < nk; s++) {
        // as gemm_tile_dl: tile s is in once this wave's loads are done and
        // every wave is past the barrier, which also ends the reads of the
        // stage that tile s+1 overwrites
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 1 < nk) issue(s + 1);
        const float *st = smem + (s % NS) * STAGE, *sb = st + TM * BK;
        floatx4 a[4][FM], b[4][FN];
#pragma unroll
        for (int q = 0; q < 4; q++) {
#pragma unroll
            for (int f = 0; f < FM; f++) a[q][f] = rd(st, wm * (TM / WM) + f * 32 + li, q);
#pragma unroll
            for (int h = 0; h < FN; h++) b[q][h] = rd(sb, wn * (TN / WN) + h * 32 + li, q);
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int ss = 0; ss < 4; ss++)
#pragma unroll
                for (int f = 0; f < FM; f++)
#pragma unroll
                    for (int h = 0; h < FN; h++)
                        acc[f][h] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q][f][ss], b[q][h][ss], acc[f][h], 0, 0, 0);
    }
    // C, or this split's partial product (partial + z*M*N, ld N)
    const int mb = m0 + wm * (TM / WM), nb = n0 + wn * (TN / WN);
    const bool part = g.partial != nullptr, accum = !part && g.accumulate;
    float *const out = part ? g.partial + (long)z * g.M * g.N : g.C;
    const long ldo = part ? (long)g.N : g.ldc;
    if (!(ldo & 3) && !((uintptr_t)out & 15) && (!accum || !((uintptr_t)g.Cin & 15))) {
        // Each wave stages RP rows x W columns at a time in its own LDS
        // region (the stage buffers are free once every wave is past the
        // loop) and stores whole rows, a float4 per lane.
        constexpr int W = FN * 32, P = W + 4, RP = NW * 32 * P <= NS * STAGE ? 32 : 16;
        static_assert(NW * RP * P <= NS * STAGE, "store staging");
        __syncthreads();
        float *T = smem + wave * RP * P;
#pragma unroll
        for (int f = 0; f < FM; f++) {
#pragma unroll
            for (int p = 0; p < 32 / RP; p++) {
                // components v of rows [p*RP, p*RP + RP) (a wave's LDS
                // operations complete in order, so this pass's reads are
                // done before the next pass overwrites the region)
#pragma unroll
                for (int h = 0; h < FN; h++)
#pragma unroll
                    for (int v = p * RP / 2; v < (p + 1) * RP / 2; v++)
                        T[((v >> 2) * 8 + 4 * lh + (v & 3) - p * RP) * P + h * 32 + li] = acc[f][h][v];
                for (int e4 = lane; e4 < RP * W / 4; e4 += 64) {
                    const int r = e4 / (W / 4), c = 4 * (e4 % (W / 4));
                    const floatx4 val = *reinterpret_cast<const floatx4 *>(T + r * P + c);
                    const int m = mb + f * 32 + p * RP + r, n = nb + c;
                    if (m >= g.M) continue;
                    const long o = (long)m * ldo + n;
                    if (n + 3 < g.N) {
                        floatx4 cv = val;
                        if (accum) cv += *reinterpret_cast<const floatx4 *>(g.Cin + o);
                        *reinterpret_cast<floatx4 *>(out + o) = cv;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (n + e < g.N) out[o + e] = accum ? g.Cin[o + e] + val[e] : val[e];
                    }
                }
            }
        }
        return;
    }
#pragma unroll
    for (int f = 0; f < FM; f++)
#pragma unroll
        for (int h = 0; h < FN; h++) {
            const int n = nb + h * 32 + li;
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int m = mb + f * 32 + (v >> 2) * 8 + 4 * lh + (v & 3);
                if (n >= g.N || m >= g.M) continue;
                const long o = (long)m * ldo + n;
                out[o] = accum ? g.Cin[o] + acc[f][h][v] : acc[f][h][v];
            }
        }
}

// Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its
// own L2.  Block b runs tile xcd_tile(b): XCD c gets the c-th contiguous
// range of the tiles, in order, so tiles that read the same operand tile
// run together on one XCD and fetch it into that L2 once.
__device__ __forceinline__ int xcd_tile(int b, int total) {
    const int q = total >> 3, r = total & 7, c = b & 7;
    return c * q + min(c, r) + (b >> 3);
}

// Grids of kXcdGrid blocks and more take tiles in xcd_tile order: split
// index slowest; within a split, neighbouring tiles share the tile of the
// larger operand (A's rows when M > N, else B's columns).  Smaller grids
// (at most a few blocks per CU, no reuse to gain) keep the grid's order.
template <bool AT, bool BT, int TM, int TN, int P, bool VEC, int EPI = GEMM_EPI_NONE, int NORM = 0>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g) {
    const int gx = gridDim.x, gy = gridDim.y, per_z = gx * gy, total = per_z * gridDim.z;
    int m = blockIdx.y, n = blockIdx.x, z = blockIdx.z;
    if (total >= kXcdGrid) {                                        // uniform
        const int t = xcd_tile(blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z), total);
        z = t / per_z;
        const int u = t - z * per_z;
        if (g.M > g.N) m = u / gx, n = u - m * gx;
        else n = u / gy, m = u - n * gy;
    }
    gemm_tile<AT, BT, TM, TN, P, VEC, EPI, NORM>(g, m * TM, n * TN, z);
}

// The direct-to-LDS GEMM (grid and tile order as k_gemm).
template <bool AK, bool BKM, int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_dl(GemmArgs g) {
    const int gx = gridDim.x, gy = gridDim.y, per_z = gx * gy, total = per_z * gridDim.z;
    int m = blockIdx.y, n = blockIdx.x, z = blockIdx.z;
    if (total >= kXcdGrid) {                                        // uniform
        const int t = xcd_tile(blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z), total);
        z = t / per_z;
        const int u = t - z * per_z;
        if (g.M > g.N) m = u / gx, n = u - m * gx;
        else n = u / gy, m = u - n * gy;
    }
    gemm_tile_dl<AK, BKM, TM, TN, WM, WN>(g, m * TM, n * TN, z);
}

// The classifier's NT forward on the 32x32x2 tiles (grid and tile order as k_gemm).
template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_dl32(GemmArgs g) {
    const int gx = gridDim.x, gy = gridDim.y, per_z = gx * gy, total = per_z * gridDim.z;
    int m = blockIdx.y, n = blockIdx.x, z = blockIdx.z;
    if (total >= kXcdGrid) {                                        // uniform
        const int t = xcd_tile(blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z), total);
        z = t / per_z;
        const int u = t - z * per_z;
        if (g.M > g.N) m = u / gx, n = u - m * gx;
        else n = u / gy, m = u - n * gy;
    }
    gemm_tile_dl32<TM, TN, WM, WN>(g, m * TM, n * TN, z);
}

// The per-layer panel GEMM (grid and tile order as k_gemm).
template <bool BKM, int NSK, int EPI>
__global__ __launch_bounds__(256) void k_gemm_panel(GemmArgs g) {
    const int gx = gridDim.x, gy = gridDim.y, per_z = gx * gy, total = per_z * gridDim.z;
    int m = blockIdx.y, n = blockIdx.x, z = blockIdx.z;
    if (total >= kXcdGrid) {                                        // uniform
        const int t = xcd_tile(blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z), total);
        z = t / per_z;
        const int u = t - z * per_z;
        if (g.M > g.N) m = u / gx, n = u - m * gx;
        else n = u / gy, m = u - n * gy;
    }
    gemm_tile_panel<BKM, NSK, EPI>(g, m * 32, n * 32, z);
}

// Grouped TN GEMMs (32x32 tiles, whole K): block b runs tile
// t = xcd_tile(b) - d.tile0 of the descriptor d whose tile range holds it;
// tiles run along N first, so neighbours share the A^T tile.  The launch
// covers entries [i0, i1) of the table, whose tiles start at d[i0].tile0 (a
// tile's result does not depend on the block that computes it, so a launch
// of a sub-range gives the same bits as the whole table).
template <int TM, int TN, bool VEC>
__global__ __launch_bounds__(256) void k_gemm_tn_group(const GemmGroupDesc *d, int i0, int i1) {
    const int b = d[i0].tile0 + xcd_tile(blockIdx.x, gridDim.x);
    int i = i0;
    while (i + 1 < i1 && d[i + 1].tile0 <= b) i++;
    const GemmGroupDesc &e = d[i];
    const int t = b - e.tile0;
    gemm_tile<true, false, TM, TN, kRing32, VEC>(e.g, (t / e.tiles_n) * TM, (t % e.tiles_n) * TN, 0);
}

// C = (Cin +) sum_z partial[z], z ascending.
__global__ __launch_bounds__(256) void k_splitk_reduce(const float *partial, int splits, float *C, const float *Cin,
                                                       long ldc, int M, int N, int accumulate) {
    const long idx = (long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long)M * N) return;
    const int m = (int)(idx / N), n = (int)(idx % N);
    const float s = sum_splits(partial, splits, (long)M * N, idx);
    const long o = (long)m * ldc + n;
    C[o] = accumulate ? Cin[o] + s : s;
}

inline bool al16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

bool gemm_big_tiles(int op, int M, int N, int K) { return K >= 4096 || (op == 2 && (long)M * N >= (4L << 20)); }

// How launch_gemm splits K: `chosen` splits fit the workspace, then K is
// cut into whole K steps per split, which gives `splits` (<= chosen).
struct SplitPlan { int chosen, splits, k_per_split; };
SplitPlan split_plan(int op, int M, int N, int K, size_t ws_floats, int ek) {
    if (ek != GEMM_EPI_NONE) return SplitPlan{1, 1, K};          // the epilogue needs whole-K sums
    const bool big = gemm_big_tiles(op, M, N, K);
    const int T = big ? 64 : 32;
    const long blocks = (long)((N + T - 1) / T) * ((M + T - 1) / T);
    const int nk = (K + BK - 1) / BK;
    int splits = 1;
    if (big && K >= 4096 && blocks < 512) splits = (int)std::min<long>((1024 + blocks - 1) / blocks, nk / 8);
    else if (!big && blocks < 128 && nk > 9) splits = std::min(8, nk / 8);
    while (splits > 1 && (size_t)splits * M * N > ws_floats) splits--;
    const int chosen = std::max(1, splits);
    const int kps = ((K + chosen - 1) / chosen + BK - 1) / BK * BK;
    return SplitPlan{chosen, (K + kps - 1) / kps, kps};
}

}  // namespace

bool gemm_norm_fusable(int M, int N, int K, const float *A, long lda, const float *B, long ldb, int epi_kind,
                       const GemmNorm &nm) {
    if (nm.kind < GEMM_NORM_PLAIN || nm.kind > GEMM_NORM_EMBED || !nm.w || !nm.xn_out) return false;
    if (epi_kind != GEMM_EPI_ROPE && epi_kind != GEMM_EPI_SWIGLU) return false;
    if (M <= 0 || N <= 0 || K <= 0 || K % 4 || lda != K || ldb % 4 || ldb < K || gemm_big_tiles(2, M, N, K)) return false;
    if (!A || !B || !al16(A) || !al16(B) || !al16(nm.w) || !al16(nm.xn_out)) return false;
    if (nm.kind != GEMM_NORM_PLAIN && (!nm.x_out || !al16(nm.x_out))) return false;
    if (nm.kind == GEMM_NORM_SPLITS &&
        (nm.pk.splits < 1 || nm.pk.splits > kNormSplits || !nm.pk.parts || !al16(nm.pk.parts) || nm.pk.stride % 4 ||
         nm.pk.stride < (long)M * K || (nm.cin && !al16(nm.cin))))
        return false;
    if (nm.kind == GEMM_NORM_EMBED && (!nm.tok || !nm.emb || !nm.tok_bits || !al16(nm.emb))) return false;
    return true;
}

size_t gemm_workspace_floats(int op, int M, int N, int K, size_t ws_floats) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const SplitPlan p = split_plan(op, M, N, K, ws_floats, GEMM_EPI_NONE);
    return p.chosen > 1 ? (size_t)p.chosen * M * N : 0;
}

// Launch op(A).op(B) with shapes validated; `ws` (optional) is a split-K
// workspace of ws_floats floats.
int launch_gemm(int op, const float *A, long lda, const float *B, long ldb, float *C, long ldc, int M, int N,
                int K, int accumulate, float *ws, size_t ws_floats, hipStream_t s, const float *Cin, SplitK *defer,
                const GemmEpi *epi, const GemmNorm *norm) {
    if (defer) *defer = SplitK{nullptr, 0, 0};
    const int ek = epi ? epi->kind : GEMM_EPI_NONE;
    const int nk_kind = norm ? norm->kind : 0;
    if (nk_kind && (op != 2 || accumulate || !gemm_norm_fusable(M, N, K, A, lda, B, ldb, ek, *norm)))
        return set_error(PTMI_ERR_ARG, "gemm: the fused norm does not fit this GEMM");
    if (ek == GEMM_EPI_SWIGLU_BWD ? (op != 0 || !epi->out || !epi->out2 || !epi->aux)
                                  : ek != GEMM_EPI_NONE && (op != 2 || N % 2 || (ek == GEMM_EPI_SWIGLU && !epi->out) ||
                                                            (ek == GEMM_EPI_ROPE && (epi->rope_dim % 2 || epi->head_dim <= 0))))
        return set_error(PTMI_ERR_ARG, "gemm: fused epilogue %d does not fit this GEMM", ek);
    if (M <= 0 || N <= 0 || K <= 0) return set_error(PTMI_ERR_ARG, "gemm: M=%d N=%d K=%d", M, N, K);
    if (!A || !B || !C) return set_error(PTMI_ERR_ARG, "gemm: null operand");
    if (op < 0 || op > 2) return set_error(PTMI_ERR_ARG, "gemm: op %d", op);
    const bool AT = op == 1, BT = op == 2;
    // minimum leading dimensions
    if ((AT ? lda < M : lda < K) || (BT ? ldb < K : ldb < N) || ldc < N)
        return set_error(PTMI_ERR_ARG, "gemm: leading dimension too small");
    GemmArgs g;
    g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.C = C; g.ldc = ldc;
    g.M = M; g.N = N; g.K = K; g.accumulate = accumulate;
    g.Cin = Cin ? Cin : C;
    g.upd = nullptr; g.lr = nullptr; g.keep = nullptr;
    // float4 loads when both operands have aligned rows and a contiguous
    // extent that is a multiple of 4 (M for A^T, K for A; K for B^T, N for B)
    const bool vec = al16(A) && lda % 4 == 0 && (AT ? M : K) % 4 == 0 && al16(B) && ldb % 4 == 0 &&
                     (BT ? K : N) % 4 == 0;
    // Kernel choice, measured on MI355X for the training shapes (graph-
    // replayed launches): 32x32 tiles win everywhere except long K (>= 4096:
    // 64x64 with K split over >= 512 blocks) and large NT outputs (>= 4M
    // elements: 64x64).  Every small GEMM is bound by the latency of its K
    // steps, so K is split when a 32x32 grid is small and K long: about
    // eight K steps per split (K=768: 3 splits, K=864: 3, K=1536: 6).  With
    // the panel kernel taking up to 9 K steps at once, eight per split ran
    // the stories15M T=256 step in 0.769-0.771 ms against 0.778-0.783 with
    // six (12.9 us less kernel time per step); nine and ten were no faster.
    const bool big = gemm_big_tiles(op, M, N, K);
    const int TM = big ? 64 : 32, TN = TM;
    const int gx = (N + TN - 1) / TN, gy = (M + TM - 1) / TM;
    const SplitPlan plan = split_plan(op, M, N, K, ws_floats, ek);
    int splits = plan.splits;
    g.k_per_split = plan.k_per_split;
    g.partial = splits > 1 ? ws : nullptr;
    g.epi = epi ? *epi : GemmEpi{};
    g.nrm = norm ? *norm : GemmNorm{};
    if (gy > 65535) return set_error(PTMI_ERR_ARG, "gemm: M too large");
    dim3 grid(gx, gy, splits);
    using KFn = void (*)(GemmArgs);
    static const KFn kernels[2][2][3] = {
        {{k_gemm<false, false, 32, 32, kRing32, false>, k_gemm<true, false, 32, 32, kRing32, false>,
          k_gemm<false, true, 32, 32, kRing32, false>},
         {k_gemm<false, false, 32, 32, kRing32, true>, k_gemm<true, false, 32, 32, kRing32, true>,
          k_gemm<false, true, 32, 32, kRing32, true>}},
        {{k_gemm<false, false, 64, 64, kRing64, false>, k_gemm<true, false, 64, 64, kRing64, false>,
          k_gemm<false, true, 64, 64, kRing64, false>},
         {k_gemm<false, false, 64, 64, kRing64, true>, k_gemm<true, false, 64, 64, kRing64, true>,
          k_gemm<false, true, 64, 64, kRing64, true>}}};
    KFn fn = kernels[big][vec][op];
    if (ek != GEMM_EPI_NONE) {
        static const KFn fused[2][2][2] = {
            {{k_gemm<false, true, 32, 32, kRing32, false, GEMM_EPI_ROPE>, k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_ROPE>},
             {k_gemm<false, true, 64, 64, kRing64, false, GEMM_EPI_ROPE>, k_gemm<false, true, 64, 64, kRing64, true, GEMM_EPI_ROPE>}},
            {{k_gemm<false, true, 32, 32, kRing32, false, GEMM_EPI_SWIGLU>, k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_SWIGLU>},
             {k_gemm<false, true, 64, 64, kRing64, false, GEMM_EPI_SWIGLU>, k_gemm<false, true, 64, 64, kRing64, true, GEMM_EPI_SWIGLU>}}};
        static const KFn fused_nn[2][2] = {
            {k_gemm<false, false, 32, 32, kRing32, false, GEMM_EPI_SWIGLU_BWD>,
             k_gemm<false, false, 32, 32, kRing32, true, GEMM_EPI_SWIGLU_BWD>},
            {k_gemm<false, false, 64, 64, kRing64, false, GEMM_EPI_SWIGLU_BWD>,
             k_gemm<false, false, 64, 64, kRing64, true, GEMM_EPI_SWIGLU_BWD>}};
        fn = ek == GEMM_EPI_SWIGLU_BWD ? fused_nn[big][vec] : fused[ek == GEMM_EPI_SWIGLU][big][vec];
    }
    if (nk_kind) {                                       // fusable: 32x32 float4 tiles, whole K
        static const KFn fused_norm[2][3] = {
            {k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_ROPE, GEMM_NORM_PLAIN>,
             k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_ROPE, GEMM_NORM_SPLITS>,
             k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_ROPE, GEMM_NORM_EMBED>},
            {k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_SWIGLU, GEMM_NORM_PLAIN>,
             k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_SWIGLU, GEMM_NORM_SPLITS>,
             k_gemm<false, true, 32, 32, kRing32, true, GEMM_EPI_SWIGLU, GEMM_NORM_EMBED>}};
        if (big || !vec || splits != 1) return set_error(PTMI_ERR_STATE, "gemm: fused norm without whole-K float4 tiles");
        fn = fused_norm[ek == GEMM_EPI_SWIGLU][nk_kind - 1];
    }
    int threads = 256;
    // Per-layer 32x32 GEMMs with at most 9 K tiles per split: the panel
    // kernel, every K tile in flight at once.  PTMI_GEMM_PANEL is a bit mask
    // of the GEMMs that take it: 1 NT, 2 NN with the SwiGLU backward
    // epilogue, 4 the other NN (default 3).  Measured in the stories15M T=256
    // training step (kernel µs per step, eager trace): NT Wo + w2 72.8 ->
    // 70.4, QKV 37.8 -> 37.0, d_sh 45.2 -> 40.2; the split-K NN (w1|w3 and
    // QKV dX) 82.0 -> 90.9, so those keep the ring.  Graph-mode step
    // 0.780-0.785 ms against 0.787-0.796 (mask 0) and 0.790-0.795 (mask 7).
    static const int use_panel = [] { const char *e = getenv("PTMI_GEMM_PANEL"); return e ? atoi(e) & 7 : 3; }();
    const int nk_split = (plan.k_per_split + BK - 1) / BK;
    const int panel_bit = op == 2 ? 1 : ek == GEMM_EPI_SWIGLU_BWD ? 2 : 4;
    if ((use_panel & panel_bit) && !big && vec && !nk_kind && op != 1 && nk_split <= 9) {
        using PFn = void (*)(GemmArgs);
        static const PFn panel[2][2][4] = {
            {{k_gemm_panel<false, 6, GEMM_EPI_NONE>, k_gemm_panel<false, 6, GEMM_EPI_ROPE>,
              k_gemm_panel<false, 6, GEMM_EPI_SWIGLU>, nullptr},
             {k_gemm_panel<false, 9, GEMM_EPI_NONE>, k_gemm_panel<false, 9, GEMM_EPI_ROPE>,
              k_gemm_panel<false, 9, GEMM_EPI_SWIGLU>, nullptr}},
            {{k_gemm_panel<true, 6, GEMM_EPI_NONE>, nullptr, nullptr, k_gemm_panel<true, 6, GEMM_EPI_SWIGLU_BWD>},
             {k_gemm_panel<true, 9, GEMM_EPI_NONE>, nullptr, nullptr, k_gemm_panel<true, 9, GEMM_EPI_SWIGLU_BWD>}}};
        const int ei = ek == GEMM_EPI_NONE ? 0 : ek == GEMM_EPI_ROPE ? 1 : ek == GEMM_EPI_SWIGLU ? 2 : 3;
        const PFn pf = panel[op == 0][nk_split > 6][ei];
        if (pf) fn = pf;
    }
    // The large whole-K GEMMs without a fused epilogue (the classifier's
    // forward and weight gradient) take the direct-to-LDS tiles.
    if (vec && ek == GEMM_EPI_NONE && splits == 1 && (long)M * N >= (4L << 20)) {
        if (op == 2 && M >= 192) {
            grid = dim3((unsigned)((N + 127) / 128), (unsigned)((M + 255) / 256), 1);
            fn = k_gemm_dl32<256, 128, 4, 2>;
            threads = 512;
        } else if (op == 1) {
            grid = dim3((unsigned)((N + 95) / 96), (unsigned)((M + 127) / 128), 1);
            fn = k_gemm_dl<true, true, 128, 96, 4, 2>;
            threads = 512;
        }
    }
    hipLaunchKernelGGL(fn, grid, dim3(threads), 0, s, g);
    PTMI_HIP(hipGetLastError());
    if (splits > 1 && defer) {
        *defer = SplitK{ws, splits, (long)M * N};
    } else if (splits > 1) {
        const long n = (long)M * N;
        hipLaunchKernelGGL(k_splitk_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ws, splits, C, g.Cin,
                           ldc, M, N, accumulate);
        PTMI_HIP(hipGetLastError());
    }
    return PTMI_OK;
}

size_t gemm_group_desc_bytes(int n) { return sizeof(GemmGroupDesc) * (size_t)n; }

int gemm_tn_group_prepare(const TnGemm *list, int n, const float *lr, void *host_desc, int *tiles_total,
                          int *vec_out) {
    GemmGroupDesc *d = static_cast<GemmGroupDesc *>(host_desc);
    int t = 0, vec = 1;
    for (int i = 0; i < n; i++) {
        const TnGemm &e = list[i];
        if (e.M <= 0 || e.N <= 0 || e.K <= 0 || !e.A || !e.B || !e.C || e.lda < e.M || e.ldb < e.N || e.ldc < e.N)
            return set_error(PTMI_ERR_ARG, "grouped gemm %d: bad shape", i);
        GemmArgs &g = d[i].g;
        g = GemmArgs{};
        g.A = e.A; g.lda = e.lda; g.B = e.B; g.ldb = e.ldb; g.C = e.C; g.ldc = e.ldc; g.Cin = e.C;
        g.M = e.M; g.N = e.N; g.K = e.K; g.accumulate = 0; g.partial = nullptr; g.k_per_split = e.K;
        if (e.upd && !lr) return set_error(PTMI_ERR_ARG, "grouped gemm %d: update without a learning rate", i);
        g.upd = e.upd; g.lr = lr; g.keep = e.keep;
        if (!(al16(e.A) && e.lda % 4 == 0 && e.M % 4 == 0 && al16(e.B) && e.ldb % 4 == 0 && e.N % 4 == 0)) vec = 0;
        d[i].tiles_n = (e.N + 31) / 32;
        d[i].tile0 = t;
        t += d[i].tiles_n * ((e.M + 31) / 32);
    }
    *tiles_total = t;
    *vec_out = vec;
    return PTMI_OK;
}

int launch_gemm_tn_group(const void *dev_desc, int i0, int i1, int tiles, int vec, hipStream_t s) {
    if (i1 <= i0 || tiles <= 0) return PTMI_OK;
    void (*fn)(const GemmGroupDesc *, int, int) = vec ? k_gemm_tn_group<32, 32, true> : k_gemm_tn_group<32, 32, false>;
    hipLaunchKernelGGL(fn, dim3((unsigned)tiles), dim3(256), 0, s, static_cast<const GemmGroupDesc *>(dev_desc), i0, i1);
    PTMI_HIP(hipGetLastError());
    return PTMI_OK;
}

}  // namespace ptmi

using namespace ptmi;

namespace {

// Host-pointer GEMM: upload, run, download (the drop-in replacements for
// the reference's host-memory GEMM calls).
int host_gemm(int op, const float *A, size_t a_n, long lda, const float *B, size_t b_n, long ldb, float *C, int M,
              int N, int K, int accumulate) {
    int st = ensure_init();
    if (st) return st;
    hipStream_t s = lib_stream();
    const size_t c_n = (size_t)M * N;
    const size_t ws_n = std::min<size_t>(c_n * 64, (size_t)64 << 20);
    float *dA = scratch_buf(0, a_n + b_n + c_n);
    float *ws = scratch_buf(3, ws_n);
    if (!dA || !ws) return ptmi_last_status();
    float *dB = dA + a_n, *dC = dB + b_n;
    PTMI_HIP(hipMemcpyAsync(dA, A, a_n * sizeof(float), hipMemcpyHostToDevice, s));
    PTMI_HIP(hipMemcpyAsync(dB, B, b_n * sizeof(float), hipMemcpyHostToDevice, s));
    if (accumulate) PTMI_HIP(hipMemcpyAsync(dC, C, c_n * sizeof(float), hipMemcpyHostToDevice, s));
    if ((st = launch_gemm(op, dA, lda, dB, ldb, dC, N, M, N, K, accumulate, ws, ws_n, s))) return st;
    PTMI_HIP(hipMemcpyAsync(C, dC, c_n * sizeof(float), hipMemcpyDeviceToHost, s));
    PTMI_HIP(hipStreamSynchronize(s));
    return PTMI_OK;
}

}  // namespace

namespace ptmi {

// Split-K workspace of ptmi_gemm_dev: up to 64 partial products, at most
// 256 MiB.
size_t gemm_dev_ws_floats(int M, int N) {
    if (M <= 0 || N <= 0) return 0;
    return std::min<size_t>((size_t)M * N * 64, (size_t)64 << 20);
}

// ── the entry point that allocates nothing ───────────────────────────────
// ptmi_gemm_dev_noalloc keeps its split-K partials in this file-scope
// device array (16 MiB; each GPU the library runs on holds it until the
// process ends).  In host code `scratch` names a host-side stand-in, not
// device memory: the device address comes from hipGetSymbolAddress, once
// per device at ptmi_init, and only that address is handed to kernels.
constexpr size_t kNoAllocScratchFloats = (size_t)4 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];
static float *g_scratch_dev[kMaxDevices] = {};

int gemm_scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices)
        return set_error(PTMI_ERR_ARG, "device %d: no GEMM scratch slot", device);
    if (g_scratch_dev[device]) return PTMI_OK;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_check(e, "hipGetSymbolAddress(scratch)");
    if (!p) return set_error(PTMI_ERR_HIP, "hipGetSymbolAddress(scratch) gave no address");
    g_scratch_dev[device] = static_cast<float *>(p);
    return PTMI_OK;
}

}  // namespace ptmi

extern "C" {

int ptmi_gemm_dev_noalloc(int op, const float *dA, long lda, const float *dB, long ldb, float *dC, long ldc, int M,
                          int N, int K, int accumulate, void *stream) {
    if (!lib_initialised())
        return set_error(PTMI_ERR_STATE, "ptmi_gemm_dev_noalloc: call ptmi_init first (it locates the scratch)");
    float *ws = g_scratch_dev[lib_device()];
    if (!ws) return set_error(PTMI_ERR_STATE, "ptmi_gemm_dev_noalloc: no scratch on device %d", lib_device());
    // The K split ptmi_gemm_dev would take must fit the fixed scratch, so
    // both entries sum in the same order and give the same bits.
    const size_t need = gemm_workspace_floats(op, M, N, K, gemm_dev_ws_floats(M, N));
    if (need > kNoAllocScratchFloats)
        return set_error(PTMI_ERR_ARG,
                         "ptmi_gemm_dev_noalloc: %dx%dx%d needs %zu floats of split-K partials; the fixed scratch "
                         "holds %zu",
                         M, N, K, need, kNoAllocScratchFloats);
    // the split is chosen from ptmi_gemm_dev's workspace size, not the
    // scratch's, so that both take the same number of splits
    return launch_gemm(op, dA, lda, dB, ldb, dC, ldc, M, N, K, accumulate, ws,
                       std::min(kNoAllocScratchFloats, gemm_dev_ws_floats(M, N)),
                       stream ? (hipStream_t)stream : lib_stream());
}

int ptmi_gemm_dev(int op, const float *dA, long lda, const float *dB, long ldb, float *dC, long ldc, int M, int N,
                  int K, int accumulate, void *stream) {
    int st = ensure_init();
    if (st) return st;
    const size_t ws_n = gemm_dev_ws_floats(M, N);
    float *ws = scratch_buf(3, ws_n);
    if (!ws) return ptmi_last_status();
    return launch_gemm(op, dA, lda, dB, ldb, dC, ldc, M, N, K, accumulate, ws, ws_n,
                       stream ? (hipStream_t)stream : lib_stream());
}

int ptmi_sgemm_rect(const float *A, const float *B, float *C, int M, int K, int N, int accumulate) {
    if (!A || !B || !C || M <= 0 || N <= 0 || K <= 0)
        return set_error(PTMI_ERR_ARG, "ptmi_sgemm_rect: bad arguments (M=%d K=%d N=%d)", M, K, N);
    return host_gemm(0, A, (size_t)M * K, K, B, (size_t)K * N, N, C, M, N, K, accumulate);
}

int ptmi_matmul_backward_weight_batched_checked(float *d_W, const float *d_y_all, const float *x_all, int out_dim,
                                                int in_dim, int T) {
    if (!d_W || !d_y_all || !x_all || out_dim <= 0 || in_dim <= 0 || T < 0)
        return set_error(PTMI_ERR_ARG, "ptmi_matmul_backward_weight_batched: bad arguments");
    if (T == 0) return PTMI_OK;
    // dW[out,in] += dY[T,out]^T . X[T,in]   (TN: A stored [K=T][M=out])
    return host_gemm(1, d_y_all, (size_t)T * out_dim, out_dim, x_all, (size_t)T * in_dim, in_dim, d_W, out_dim, in_dim,
                     T, 1);
}

int ptmi_matmul_backward_input_batched(float *d_x_all, const float *W, const float *d_y_all, int out_dim, int in_dim,
                                       int T, int accumulate) {
    if (!d_x_all || !W || !d_y_all || out_dim <= 0 || in_dim <= 0 || T < 0)
        return set_error(PTMI_ERR_ARG, "ptmi_matmul_backward_input_batched: bad arguments");
    if (T == 0) return PTMI_OK;
    // dX[T,in] (+)= dY[T,out] . W[out,in]   (NN)
    return host_gemm(0, d_y_all, (size_t)T * out_dim, out_dim, W, (size_t)out_dim * in_dim, in_dim, d_x_all, T, in_dim,
                     out_dim, accumulate);
}

// The reference's void entries report failure by panicking
// (libpi/libc/demand.h:20-60): message on stderr, then abort().
static void panic_on(int st, const char *what) {
    if (st == PTMI_OK) return;
    fprintf(stderr, "%s: %s\n", what, ptmi_last_error());
    abort();
}

void ptmi_sgemm_rect_tmu(const float *A, const float *B, float *C, int M, int K, int N, int num_qpus,
                         int accumulate) {
    // num_qpus selects no resource here, but keeps the reference's range
    // check (gemm_rect.c:34: 1..12); N needs no multiple of 16 (:33).
    if (num_qpus < 1 || num_qpus > 12)
        panic_on(set_error(PTMI_ERR_ARG, "num_qpus %d outside 1..12", num_qpus), "ptmi_sgemm_rect_tmu");
    panic_on(ptmi_sgemm_rect(A, B, C, M, K, N, accumulate), "ptmi_sgemm_rect_tmu");
}

void ptmi_sgemm_cpu(const float *A, const float *B, float *C, int M, int K, int N) {
    panic_on(ptmi_sgemm_rect(A, B, C, M, K, N, 0), "ptmi_sgemm_cpu");
}

void ptmi_matmul_backward_weight_batched(float *d_W, const float *d_y_all, const float *x_all, int out_dim,
                                         int in_dim, int T) {
    panic_on(ptmi_matmul_backward_weight_batched_checked(d_W, d_y_all, x_all, out_dim, in_dim, T),
             "ptmi_matmul_backward_weight_batched");
}

}  // extern "C"
