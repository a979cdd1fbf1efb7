// Per-channel (vector) gates on the chunked form, bf16 inputs: one decay d_tj per key channel j (GATE_DECAY_VEC,
// tools/gdn_vjp.py:174-179 with a [B,T,Hv,Dk] gate; or its log, GATE_LOG_VEC, with dg returned for the log).  Per 64-token chunk of one value head, with G_rj the cumulative
// log decay of channel j up to token r (G_C its last row) and E_rsj = exp(G_rj - G_sj):
//   A_rs = beta_r sum_j k_rj k_sj E_rsj (s < r),   P_rs = sum_j q_rj k_sj E_rsj (s <= r),   T = (I + A)^-1
//   W = T diag(beta) (K * exp(G)),   U = T diag(beta) V,   Delta = U - W h
//   Y = (Q * exp(G)) h + P Delta,   h' = diag(exp(G_C)) h + (K * exp(G_C - G))^T Delta
// which is the token recurrence in exact arithmetic (tests/chunk_model.py states it and its VJP).  The sequential
// kernels are the scalar-gate bf16 ones with the VG flag (gdn_chunk.hip): they read the decayed operands written
// here instead of scaling rows.  This file holds the two chunk-parallel stages:
//   ck_prep_vg        grid (NC, Hv, B): G, A, P, T, W, U and the operand tiles of one chunk-head.
//   ck_bwd_local_vg   grid (NC, Hk, B): the chunk's dq, dk, dv, dbeta and per-channel dg, for the value heads of a
//                     key head in turn.
// The pair sums over channels cannot be one product of K exp(G) and K exp(-G): exp(-G_s) overflows over a chunk.
// They are formed per pair of 16-token blocks R > S through the last token b = 16R - 1 of the block before R,
//   M_RS = (X_R * exp(G_R - G_b)) (Y_S * exp(G_b - G_S))^T,
// where both factors are <= 1, and elementwise on the four diagonal blocks.  G is kept in log2 units so that every
// factor is one v_exp_f32.
#include "gdn_chunk_common.h"

namespace gdn {
namespace ck {

constexpr int SB = 16;  // token block of the pair sums

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Sum over the 8 lanes of an aligned group (lane bits 0-2): every lane of the group receives the total.
__device__ __forceinline__ float group8_sum(float x) {
    x += dpp_mov<DPP_QUAD_1032>(x);
    x += dpp_mov<DPP_QUAD_2301>(x);
    x += dpp_mov<DPP_ROW_HALF_MIRROR>(x);
    return x;
}

// 8 consecutive bf16 of a tile as floats.
__device__ __forceinline__ void ld8(const bfr *p, float (&x)[8]) {
    const uint4 v = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = bf2f(w[i] & 0xffffu);
        x[2 * i + 1] = bf2f(w[i] >> 16);
    }
}
__device__ __forceinline__ void ld8(const float *p, float (&x)[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
    return make_uint4(pk(x[0], x[1]), pk(x[2], x[3]), pk(x[4], x[5]), pk(x[6], x[7]));
}
// hi = bf16(x), lo = bf16(x - hi) of 8 values as MFMA fragments
__device__ __forceinline__ void split8(const float (&x)[8], bf8 &hi, bf8 &lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        hi[i] = (__bf16)x[i];
        lo[i] = (__bf16)(x[i] - (float)hi[i]);
    }
}

// ---------------------------------------------------------------------------------------------- ck_prep_vg
//
// LDS regions (bytes), time-shared:
//   R_K   K bf16 [64][VLK]                                      -> W staging (bf16 [64][VLK])
//   R_Q   Q bf16 [64][VLK] -> V^T bf16 [128][VLT]
//   R_G   G log2(e) fp32 [64][VLG]                              -> U staging (fp32 [64][VLG])
//   R_A   A fp32 [64][LDC]
//   R_T   P hi / lo staging bf16 [2][64][64] -> T fp32 [64][LDC]
//   R_KG  linear decays fp32 [64][VLG] -> (K * exp(G))^T hi / lo bf16 [2][128][VLT]
constexpr int VLK = D + 8, VLG = D + 4, VLT = C + 8;
constexpr int VP_K = 0;
constexpr int VP_Q = VP_K + C * VLK * 2;
constexpr int VP_G = VP_Q + D * VLT * 2;
constexpr int VP_A = VP_G + C * VLG * 4;
constexpr int VP_T = VP_A + C * LDC * 4;
constexpr int VP_KG = VP_T + C * LDC * 4;
constexpr int VP_END = VP_KG + 2 * D * VLT * 2;
static_assert(C * VLK * 2 <= D * VLT * 2, "Q fits the V^T region");
static_assert(2 * C * C * 2 <= C * LDC * 4, "P hi / lo staging fits the T region");
static_assert(VP_END + 3 * 256 * 4 + 4 * D * 8 + C * 4 <= 160 * 1024, "LDS");
static_assert(C * VLG * 4 <= 2 * D * VLT * 2, "the linear decays fit the (K exp(G))^T region");

// LOGG: the gates are log decays (GATE_LOG_VEC) rather than decays (GATE_DECAY_VEC)
template <bool LOGG>
__global__ __launch_bounds__(NTP) void ck_prep_vg_kernel(Args a) {
    __shared__ __align__(16) unsigned char pa[VP_END];
    __shared__ float scratch[3 * 256];
    __shared__ double sSeg[4][D];  // the four 16-token segment sums of each channel's log decays
    __shared__ float sB[C];
    bfr *const sK = reinterpret_cast<bfr *>(pa + VP_K);
    bfr *const sQ = reinterpret_cast<bfr *>(pa + VP_Q);
    bfr *const sVT = sQ;
    float *const sG = reinterpret_cast<float *>(pa + VP_G);
    float *const sA = reinterpret_cast<float *>(pa + VP_A);
    float *const sT = reinterpret_cast<float *>(pa + VP_T);
    bfr *const sPb = reinterpret_cast<bfr *>(pa + VP_T);
    bfr *const sKGh = reinterpret_cast<bfr *>(pa + VP_KG);
    bfr *const sKGl = sKGh + D * VLT;

    const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk), t0 = c * C, n = min(C, T - t0);
    const size_t ci = chunk_index(a, b, hv, c);
    const size_t qk0 = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * a.Ts + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;

    // ---- loads: V (8-token x 2-channel blocks, kept in registers), K and Q rows, beta, and the decays of channel
    // gj over tokens 16 gs .. 16 gs + 15.  Rows past n read row n - 1 and are zeroed (decay 1) after.
    static_assert((C / 8) * (D / 2) == NTP, "one V block per thread");
    const int vb = tid / (D / 2), vc = 2 * (tid - vb * (D / 2));
    uint32_t vr[8];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
        const int s2 = 8 * vb + rr;
        const uint32_t x =
            *reinterpret_cast<const uint32_t *>(static_cast<const bfr *>(a.v) + v0 + min(s2, n - 1) * v_row + vc);
        vr[rr] = s2 < n ? x : 0u;
    }
    constexpr int KPER = C * (D / 8) / NTP;
    static_assert(KPER * NTP == C * (D / 8), "even split");
    uint4 kr[KPER], qr[KPER];
#pragma unroll
    for (int p = 0; p < KPER; ++p) {
        const int pc = tid + p * NTP, r = pc / (D / 8), c8 = (pc - r * (D / 8)) * 8;
        const size_t o = qk0 + (size_t)min(r, n - 1) * qk_row + c8;
        const uint4 xk = *reinterpret_cast<const uint4 *>(static_cast<const bfr *>(a.k) + o);
        const uint4 xq = *reinterpret_cast<const uint4 *>(static_cast<const bfr *>(a.q) + o);
        kr[p] = r < n ? xk : make_uint4(0u, 0u, 0u, 0u);
        qr[p] = r < n ? xq : make_uint4(0u, 0u, 0u, 0u);
    }
    const int gj = tid & (D - 1), gs = tid >> 7;
    float gl[SB], dl[SB];  // log and linear decays (decay 1 past the sequence)
#pragma unroll
    for (int rr = 0; rr < SB; ++rr) {
        const int r = SB * gs + rr;
        const float x = a.g[(((size_t)b * a.Ts + t0 + min(r, n - 1)) * a.Hv + hv) * D + gj];
        // rows past the sequence by a 0 / 1 factor rather than a select: the compiler turned the select into a branch
        // around the gate's load, and waited there for every load in flight
        const float in = r < n ? 1.f : 0.f;
        const float l = gate_log(x, LOGG ? GATE_LOG_VEC : GATE_DECAY_VEC);
        gl[rr] = in * l;
        dl[rr] = in * (LOGG ? ex2(l * 1.4426950408889634f) : fmaxf(x, kMinDecay)) + (1.f - in);
    }
    const float b_ld = a.beta[((size_t)b * a.Ts + t0 + min(tid, n - 1)) * a.Hv + hv];
#pragma unroll
    for (int p = 0; p < KPER; ++p) {
        const int pc = tid + p * NTP, r = pc / (D / 8), c8 = (pc - r * (D / 8)) * 8;
        *reinterpret_cast<uint4 *>(sK + r * VLK + c8) = kr[p];
        *reinterpret_cast<uint4 *>(sQ + r * VLK + c8) = qr[p];
    }
    if (tid < C) sB[tid] = tid < n ? b_ld : 0.f;
    // cumulative log decays per channel: fp64 sums over each 16-token segment, then the segments' prefix
    {
        double run = 0.0;
#pragma unroll
        for (int rr = 0; rr < SB; ++rr) run += (double)gl[rr];
        sSeg[gs][gj] = run;
    }
    __syncthreads();
    {
        double run = 0.0;
        for (int s2 = 0; s2 < gs; ++s2) run += sSeg[s2][gj];
        float *const sDl = reinterpret_cast<float *>(pa + VP_KG);  // the linear decays, until (K exp(G))^T is built
#pragma unroll
        for (int rr = 0; rr < SB; ++rr) {
            run += (double)gl[rr];
            sG[(SB * gs + rr) * VLG + gj] = (float)(run * 1.4426950408889634);
            sDl[(SB * gs + rr) * VLG + gj] = dl[rr];
        }
    }
    __syncthreads();

    // ---- the decayed operand tiles and G: Q exp(G) and K exp(G_C - G) in fragment order, their transposes
    // (K exp(G_C - G))^T for the forward and (Q exp(G))^T for ck_bwd_seq, and G itself
    {
        constexpr int UPER = C * (D / 8) / NTP;  // 16-byte units per thread
#pragma unroll
        for (int p = 0; p < UPER; ++p) {
            const int u = tid + p * NTP, r = u / (D / 8), j0 = (u - r * (D / 8)) * 8;
            float kx[8], qx[8], g[8], gc[8], qg[8], kd[8];
            ld8(sK + r * VLK + j0, kx);
            ld8(sQ + r * VLK + j0, qx);
            ld8(sG + r * VLG + j0, g);
            ld8(sG + (C - 1) * VLG + j0, gc);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                qg[i] = qx[i] * ex2(g[i]);
                kd[i] = kx[i] * ex2(gc[i] - g[i]);
            }
            *reinterpret_cast<uint4 *>(a.w.QGb + ci * C * D + frag_off<D>(r, j0)) = pack8(qg);
            if (!a.fwd_only) *reinterpret_cast<uint4 *>(a.w.KDb + ci * C * D + frag_off<D>(r, j0)) = pack8(kd);
            float *gv = a.w.Gv + (ci * C + r) * D + j0;
            *reinterpret_cast<float4 *>(gv) = make_float4(g[0], g[1], g[2], g[3]);
            *reinterpret_cast<float4 *>(gv + 4) = make_float4(g[4], g[5], g[6], g[7]);
        }
#pragma unroll
        for (int p = 0; p < UPER; ++p) {
            // unit (j, r8): tokens r8 .. r8 + 7 of channel j
            const int u = tid + p * NTP, j = u % D, r8 = (u / D) * 8;
            const float gc = sG[(C - 1) * VLG + j];
            float kd[8], qg[8];
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const int r = r8 + rr;
                const float g = sG[r * VLG + j];
                kd[rr] = bf2f(sK[r * VLK + j]) * ex2(gc - g);
                qg[rr] = bf2f(sQ[r * VLK + j]) * ex2(g);
            }
            *reinterpret_cast<uint4 *>(a.w.KTb + ci * D * C + frag_off<C>(j, r8)) = pack8(kd);
            if (!a.fwd_only) *reinterpret_cast<uint4 *>(a.w.QTb + ci * D * C + frag_off<C>(j, r8)) = pack8(qg);
        }
    }

    // ---- A and P below the diagonal blocks: waves 0-5 take one block pair (R, S) each, both matrices, on split
    // operands (3 products per k-step); waves 6-7 clear the blocks above the diagonal
    if (w < 6) {
        const int R = w == 0 ? 1 : w < 3 ? 2 : 3, S = w == 0 ? 0 : w < 3 ? w - 1 : w - 3;
        const int bt = SB * R - 1, r = SB * R + li, s2 = SB * S + li;
        f4 accA = zero4(), accP = zero4();
#pragma unroll
        for (int k0 = 0; k0 < D; k0 += 32) {
            const int j0 = k0 + 8 * lg;
            float kx[8], qx[8], ks[8], gr[8], gb[8], gs8[8], xa[8], xp[8], ys[8];
            ld8(sK + r * VLK + j0, kx);
            ld8(sQ + r * VLK + j0, qx);
            ld8(sK + s2 * VLK + j0, ks);
            ld8(sG + r * VLG + j0, gr);
            ld8(sG + bt * VLG + j0, gb);
            ld8(sG + s2 * VLG + j0, gs8);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float fl = ex2(gr[i] - gb[i]), fs = ex2(gb[i] - gs8[i]);
                xa[i] = kx[i] * fl;
                xp[i] = qx[i] * fl;
                ys[i] = ks[i] * fs;
            }
            bf8 ah, al, ph, pl, bh, bl;
            split8(xa, ah, al);
            split8(xp, ph, pl);
            split8(ys, bh, bl);
            accA = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, accA, 0, 0, 0);
            accA = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, accA, 0, 0, 0);
            accA = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, accA, 0, 0, 0);
            accP = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, bh, accP, 0, 0, 0);
            accP = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, bh, accP, 0, 0, 0);
            accP = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, bl, accP, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int ro = SB * R + 4 * lg + e, so = SB * S + li;
            sA[ro * LDC + so] = sB[ro] * accA[e];
            const uint32_t h = bfbits(accP[e]);
            sPb[ro * C + so] = (bfr)h;
            sPb[C * C + ro * C + so] = (bfr)bfbits(accP[e] - bf2f(h));
        }
    } else {
        // the six 16 x 16 blocks above the diagonal blocks (S > R), 256 x 6 elements over 128 threads
        for (int i = tid - 6 * 64; i < 6 * SB * SB; i += 128) {
            const int blk = i / (SB * SB), e = i - blk * SB * SB;
            // block (R, S) with S > R: (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
            const int R = blk < 3 ? 0 : blk < 5 ? 1 : 2, S = blk < 3 ? blk + 1 : blk < 5 ? blk - 1 : 3;
            const int ro = SB * R + e / SB, so = SB * S + e % SB;
            sA[ro * LDC + so] = 0.f;
            sPb[ro * C + so] = 0;
            sPb[C * C + ro * C + so] = 0;
        }
    }
    // ---- the four diagonal blocks, elementwise, along running products of the decays: E_rs = prod_{s<u<=r} d_u.
    // Thread (block R, row pair sp, group jg of 8 channels) walks the rows r >= s of s = sp (16 - sp rows) and then
    // of s = 15 - sp (sp + 1 rows): 17 steps in every thread.  The 16 channel groups of a pair are the 16 lanes of a
    // DPP row.  The entries above the diagonal are cleared apart.
    {
        const int R = tid >> 7, sp = (tid >> 4) & 7, jg = tid & 15, j0 = 8 * jg;
        const float *const sDl = reinterpret_cast<const float *>(pa + VP_KG);
        const int s1 = SB * R + sp, s2b = SB * R + SB - 1 - sp;
        float ka[8], kb[8], E[8];
        ld8(sK + s1 * VLK + j0, ka);
        ld8(sK + s2b * VLK + j0, kb);
#pragma unroll
        for (int i = 0; i < 8; ++i) E[i] = 1.f;
        for (int it = 0; it <= SB; ++it) {
            const bool first = it < SB - sp;
            const int s2 = first ? s1 : s2b, r = first ? s1 + it : s2b + it - (SB - sp);
            float kx[8], qx[8], dr[8];
            ld8(sK + r * VLK + j0, kx);
            ld8(sQ + r * VLK + j0, qx);
            ld8(sDl + r * VLG + j0, dr);
            const bool diag = r == s2;
            float sa = 0.f, sq = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                E[i] = diag ? 1.f : E[i] * dr[i];
                const float ke = (first ? ka[i] : kb[i]) * E[i];
                sa = fmaf(kx[i], ke, sa);
                sq = fmaf(qx[i], ke, sq);
            }
            sa = row16_allreduce(sa);
            sq = row16_allreduce(sq);
            if (jg == 0) {
                sA[r * LDC + s2] = diag ? 0.f : sB[r] * sa;
                const uint32_t h = bfbits(sq);
                sPb[r * C + s2] = (bfr)h;
                sPb[C * C + r * C + s2] = (bfr)bfbits(sq - bf2f(h));
            }
        }
        for (int i = tid; i < 4 * SB * SB; i += NTP) {
            const int blk = i / (SB * SB), rl = (i / SB) % SB, sl = i % SB;
            if (sl > rl) {
                const int r = SB * blk + rl, s2 = SB * blk + sl;
                sA[r * LDC + s2] = 0.f;
                sPb[r * C + s2] = 0;
                sPb[C * C + r * C + s2] = 0;
            }
        }
    }
    __syncthreads();
    // ---- P hi / lo out in fragment order, and P^T hi / lo (the backward's A operand)
    for (int i = tid; i < 2 * C * C / 8; i += NTP) {
        const int pl = i / (C * C / 8), e0 = 8 * i - pl * C * C, m = e0 / C;
        *reinterpret_cast<uint4 *>(a.w.Pb + ci * 2 * C * C + pl * C * C + frag_off<C>(m, e0 - m * C)) =
            *reinterpret_cast<const uint4 *>(sPb + 8 * i);
    }
    if (!a.fwd_only) {
        for (int i = tid; i < 2 * C * C / 8; i += NTP) {
            // unit (s, r8) of plane pl: P[r8 .. r8 + 7][s]
            const int pl = i / (C * C / 8), u = i - pl * (C * C / 8), s2 = u % C, r8 = (u / C) * 8;
            uint32_t x[8];
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) x[rr] = sPb[pl * C * C + (r8 + rr) * C + s2];
            *reinterpret_cast<uint4 *>(a.w.PTb + ci * 2 * C * C + pl * C * C + frag_off<C>(s2, r8)) =
                make_uint4(x[0] | (x[1] << 16), x[2] | (x[3] << 16), x[4] | (x[5] << 16), x[6] | (x[7] << 16));
        }
    }
    // ---- (K exp(G))^T hi / lo (unit (j, s8)) for W; V^T into the dead Q region for U
    {
        constexpr int UPER = D * (C / 8) / NTP;
#pragma unroll
        for (int p = 0; p < UPER; ++p) {
            const int u = tid + p * NTP, j = u % D, s8 = (u / D) * 8;
            float x[8];
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) x[rr] = bf2f(sK[(s8 + rr) * VLK + j]) * ex2(sG[(s8 + rr) * VLG + j]);
            uint4 h, lo;
            pk2(x[0], x[1], h.x, lo.x);
            pk2(x[2], x[3], h.y, lo.y);
            pk2(x[4], x[5], h.z, lo.z);
            pk2(x[6], x[7], h.w, lo.w);
            *reinterpret_cast<uint4 *>(sKGh + j * VLT + s8) = h;
            *reinterpret_cast<uint4 *>(sKGl + j * VLT + s8) = lo;
        }
    }
    __syncthreads();  // P staging and Q read; the inverse overwrites the T region, V^T the Q region
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        uint32_t x[8];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) x[rr] = cc ? vr[rr] >> 16 : vr[rr] & 0xffffu;
        *reinterpret_cast<uint4 *>(sVT + (vc + cc) * VLT + 8 * vb) =
            make_uint4(x[0] | (x[1] << 16), x[2] | (x[3] << 16), x[4] | (x[5] << 16), x[6] | (x[7] << 16));
    }
    unit_lower_inverse<NTP>(sA, sT, scratch);  // ends with a barrier
    // ---- W = (T diag(beta)) (K exp(G)) (waves 0-3, both operands split), U = (T diag(beta)) V (waves 4-7)
    const int r0 = 16 * (w & 3);
    const bool isu = w >= 4;
    f4 acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = zero4();
#pragma unroll
    for (int k = 0; k < C / 32; ++k) {
        const float *tr = sT + (r0 + li) * LDC + 32 * k + 8 * lg;
        const float4 x0 = *reinterpret_cast<const float4 *>(tr), x1 = *reinterpret_cast<const float4 *>(tr + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = xv[i] * sB[32 * k + 8 * lg + i];
        bf8 ah, al;
        split8(y, ah, al);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            if (isu) {
                const bf8 vy = frag(sVT, VLT, 16 * t, 32 * k);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, vy, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, vy, acc[t], 0, 0, 0);
            } else {
                const bf8 kh = frag(sKGh, VLT, 16 * t, 32 * k), kl = frag(sKGl, VLT, 16 * t, 32 * k);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, kh, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, kh, acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, kl, acc[t], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // K, G, V^T and (K exp(G))^T read: their regions stage U (fp32, R_G) and W (bf16, R_K)
    float *const sU = sG;
    bfr *const sW = sK;
    if (isu) {
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) sU[(r0 + 4 * lg + e) * VLG + 16 * t + li] = acc[t][e];
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t wb[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wb[e] = bfbits(acc[t][e]);
                sW[(r0 + 4 * lg + e) * VLK + 16 * t + li] = (bfr)wb[e];
            }
            if (!a.fwd_only) {  // -W^T [j][r]; bf16 negation flips the sign bit
                bfr *wt = a.w.nWTb + ci * D * C + frag_off<C>(16 * t + li, r0 + 4 * lg);
                *reinterpret_cast<uint2 *>(wt) = make_uint2((wb[0] | (wb[1] << 16)) ^ 0x80008000u,
                                                            (wb[2] | (wb[3] << 16)) ^ 0x80008000u);
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < C * D / 4; i += NTP) {  // U fp32 in accumulator order: 16-byte piece i holds 4 rows
        const int blk = i >> 6, ln = i & 63, rw = 16 * (blk / (D / 16)) + 4 * (ln >> 4), cl = 16 * (blk % (D / 16)) + (ln & 15);
        *reinterpret_cast<float4 *>(a.w.U + ci * C * D + 4 * i) =
            make_float4(sU[rw * VLG + cl], sU[(rw + 1) * VLG + cl], sU[(rw + 2) * VLG + cl], sU[(rw + 3) * VLG + cl]);
    }
    for (int i = tid; i < C * D / 8; i += NTP) {  // W bf16 in fragment order
        const int r = i / (D / 8), c8 = (i - r * (D / 8)) * 8;
        *reinterpret_cast<uint4 *>(a.w.Wb + ci * C * D + frag_off<D>(r, c8)) =
            *reinterpret_cast<const uint4 *>(sW + r * VLK + c8);
    }
    if (!a.fwd_only) {  // T^T hi / lo in fragment order, as ck_prep_bf16_kernel writes it
        static_assert(C * C / 8 == NTP, "one unit per thread");
        bfr *const tb = reinterpret_cast<bfr *>(a.w.T) + ci * 2 * C * C;
        const int s2 = tid % C, r8 = (tid / C) * 8;
        float x[8];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) x[rr] = sT[(r8 + rr) * LDC + s2];
        uint4 h, lo;
        pk2(x[0], x[1], h.x, lo.x);
        pk2(x[2], x[3], h.y, lo.y);
        pk2(x[4], x[5], h.z, lo.z);
        pk2(x[6], x[7], h.w, lo.w);
        *reinterpret_cast<uint4 *>(tb + frag_off<C>(s2, r8)) = h;
        *reinterpret_cast<uint4 *>(tb + C * C + frag_off<C>(s2, r8)) = lo;
    }
}

void launch_vg_prep(const Args &a, hipStream_t st) {
    if (gate_in_log(a.gate)) hipLaunchKernelGGL(ck_prep_vg_kernel<true>, dim3(a.NC, a.Hv, a.B), dim3(NTP), 0, st, a);
    else hipLaunchKernelGGL(ck_prep_vg_kernel<false>, dim3(a.NC, a.Hv, a.B), dim3(NTP), 0, st, a);
}

// ---------------------------------------------------------------------------------------------- ck_bwd_local_vg
//
// One workgroup of 8 waves per (chunk, key head) takes the key head's value heads in turn.  Wave w owns the rows of
// token block R = w % 4 (r0 = 16 R) and the column half w / 4 of every [64][128] gradient, in MFMA accumulator
// layout, from the first products to the outputs.  With Kg = K exp(G), Kd = K exp(G_C - G), Qg = Q exp(G),
// Y2 = TdD h^T and TdD = T^T dDelta (ck_bwd_seq_bf16 with VG):
//   S1   X1 = dY h^T, Y2, X2 = Delta dh'^T, dp = dY Delta^T, dA = -(TdD Delta^T) below the diagonal, in one pass
//        over the value index (as ck_bwd_local_bf16); dv = diag(beta) TdD and rowsum(V * TdD) from the TdD loads
//   dq  = X1 exp(G) + [pair term of P, row role],  dk+ = -diag(beta) Y2 exp(G) + diag(beta) Z,
//   dk- = X2 exp(G_C - G) + [pair terms of P and of A, column role],  Z = [pair term of A with dA, row role]
//   dbeta = rowsum(V * TdD) - rowsum(Kg * Y2) + rowsum(K * Z)
//   dG  = Q * dq + K * (dk+ - dk-),   dg_log_u = sum_{r >= u} dG_r + dG_C,
//   dG_C = sum_r Kd * X2 exp... (the Kd term) + exp(G_C) rowsum(dh' * h)
// The pair terms go through the same 16-token blocks as ck_prep_vg: below the diagonal blocks on MFMA (row role of
// block R through the token before it, column role of block S through its last token, so both factors are <= 1;
// every wave contracts 48 tokens in all), on the diagonal blocks elementwise.  With decays (not log decays) the
// kernel leaves the pieces of d/d(decay) to ck_vg_dg instead of writing dg.  dq | dk of the key head are summed over
// its value heads in the part rows (fp32), each thread reading back only the elements it wrote; the last value head
// writes them in the gradient dtype.
constexpr int VSA = C * LA * 2, VSB = D * LA * 2;  // [64][136], [128][136] bf16
constexpr int VO_TD = 0, VO_DHH = VO_TD + VSA, VO_H = VO_DHH + VSB, VO_DLH = VO_H + VSB, VO_DLL = VO_DLH + VSA;
constexpr int VO_DY = VO_DLL + VSA, VARENA = VO_DY + VSA;
// after S1: the pair cotangents in both orientations (fp32 [64][LDC]) and K, Q, G with permuted columns
constexpr int VLP = D + 8, VLGp = D + 4;
constexpr int VO_DP = 0, VO_DA = VO_DP + C * LDC * 4, VO_DPT = VO_DA + C * LDC * 4, VO_DAT = VO_DPT + C * LDC * 4;
constexpr int VO_K = VO_DAT + C * LDC * 4, VO_Q = VO_K + C * VLP * 2, VO_G = VO_Q + C * VLP * 2;
constexpr int VO_END = VO_G + C * VLGp * 4;
constexpr int VO_DG = VO_DPT;  // dG fp32 [64][VLGp] over the two transposed tiles, after their last read
static_assert(VO_END <= VARENA, "second-phase tiles fit the S1 arena");
static_assert(C * VLGp * 4 <= 2 * C * LDC * 4, "dG fits the transposed pair tiles");

// Column j of a [64][128] tile at this position of the permuted tiles: the four columns 64 ch + 16 t + li (t = 0..3)
// that lane (ch, li) owns are contiguous.
__device__ __forceinline__ int pcol(int j) { return (j & ~63) + (j & 15) * 4 + ((j >> 4) & 3); }

// DEC: per-channel decays.  Their gradient d/d(decay) = dg_log / d loses every digit where d is small (dg_log is a
// suffix sum of terms that each carry the factor d), so this head writes no dg: it leaves the pieces of the pair
// terms, before their decay factors, in the vgd buffer, and ck_vg_dg forms d/d(decay) from them with factors <= 1.
template <bool DYF32, bool DEC>
__device__ __forceinline__ void bwd_local_vg_head(const Args &a, int c, int hk, int b, int rr, int rep) {
    __shared__ __align__(16) unsigned char arena[VARENA];
    __shared__ float sB[C], sVT[C], sHdot[D], sGCp[D];
    __shared__ float sRow[2][C];
    __shared__ float sDgc[4][D];
    __shared__ float sSegT[4][D];  // 16-row segment totals of dG per channel
    auto T16 = [&](int off) { return reinterpret_cast<bfr *>(arena + off); };
    auto F32 = [&](int off) { return reinterpret_cast<float *>(arena + off); };

    const bool first = rr == 0, last = rr == rep - 1;
    const int hv = hk * rep + rr;
    const int T = a.T, t0 = c * C, n = min(C, T - t0);
    float *const part_row = a.w.part + (((size_t)b * T + t0) * a.Hk + hk) * 2 * D;
    const size_t part_rs = (size_t)a.Hk * 2 * D;
    const size_t qk_out = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D;
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int R = w & 3, r0 = 16 * R, ch = w >> 2;
    const size_t ci = chunk_index(a, b, hv, c);
    float *const vgd = DEC ? a.w.vgd + ci * VGD_FLOATS : nullptr;
    const bfr *Hc = reinterpret_cast<const bfr *>(a.w.H) + ci * D * D;
    const bfr *dHc = reinterpret_cast<const bfr *>(a.w.dH) + ci * D * D;
    const float *Dc = a.w.Dl + ci * C * D;
    const float *TDc = a.w.dDl + ci * C * D;
    const size_t qk0 = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * a.Ts + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;
    const bfr *qsrc = static_cast<const bfr *>(a.q) + qk0, *ksrc = static_cast<const bfr *>(a.k) + qk0;
    const bfr *vsrc = static_cast<const bfr *>(a.v) + v0;

    // ---- S1 staging: h, dh' (and the rows of <dh', h>), Delta hi / lo, TdD, dY; dv and rowsum(V * TdD) leave from
    // the fp32 TdD loads
    {
        constexpr int SPER = D * (D / 8) / NTB, NPER = C * (D / 8) / NTB;
        static_assert(SPER * NTB == D * (D / 8) && NPER * NTB == C * (D / 8), "even split");
        uint4 hr[SPER], dhr[SPER], dl[2 * NPER], td[2 * NPER], yr[DYF32 ? 2 * NPER : NPER], vr[NPER];
        float bt[NPER];
#pragma unroll
        for (int p = 0; p < SPER; ++p) {
            hr[p] = reinterpret_cast<const uint4 *>(Hc)[tid + p * NTB];
            dhr[p] = reinterpret_cast<const uint4 *>(dHc)[tid + p * NTB];
        }
#pragma unroll
        for (int p = 0; p < NPER; ++p) {
            const int pc = tid + p * NTB, r = pc / (D / 8), c8 = (pc - r * (D / 8)) * 8;
            dl[2 * p] = *reinterpret_cast<const uint4 *>(Dc + r * D + c8);
            dl[2 * p + 1] = *reinterpret_cast<const uint4 *>(Dc + r * D + c8 + 4);
            td[2 * p] = *reinterpret_cast<const uint4 *>(TDc + r * D + c8);
            td[2 * p + 1] = *reinterpret_cast<const uint4 *>(TDc + r * D + c8 + 4);
            const int rc = min(r, n - 1);
            const uint4 xv = *reinterpret_cast<const uint4 *>(vsrc + (size_t)rc * v_row + c8);
            vr[p] = r < n ? xv : make_uint4(0u, 0u, 0u, 0u);
            const float xb = a.beta[((size_t)b * a.Ts + t0 + rc) * a.Hv + hv];
            bt[p] = r < n ? xb : 0.f;
            if constexpr (DYF32) {
                const float *ys = static_cast<const float *>(a.dy) + v0 + (size_t)rc * v_row + c8;
                const uint4 y0 = *reinterpret_cast<const uint4 *>(ys), y1 = *reinterpret_cast<const uint4 *>(ys + 4);
                yr[2 * p] = r < n ? y0 : make_uint4(0u, 0u, 0u, 0u);
                yr[2 * p + 1] = r < n ? y1 : make_uint4(0u, 0u, 0u, 0u);
            } else {
                const uint4 y0 = *reinterpret_cast<const uint4 *>(static_cast<const bfr *>(a.dy) + v0 + (size_t)rc * v_row + c8);
                yr[p] = r < n ? y0 : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        if (tid < C) {
            const float xb = a.beta[((size_t)b * a.Ts + t0 + min(tid, n - 1)) * a.Hv + hv];
            sB[tid] = tid < n ? xb : 0.f;
        }
        bfr *const th = T16(VO_H), *const tdh = T16(VO_DHH);
#pragma unroll
        for (int p = 0; p < SPER; ++p) {
            const int pc = tid + p * NTB, r = pc / (D / 8), c8 = (pc - r * (D / 8)) * 8;
            *reinterpret_cast<uint4 *>(th + r * LA + c8) = hr[p];
            *reinterpret_cast<uint4 *>(tdh + r * LA + c8) = dhr[p];
            const uint32_t hw[4] = {hr[p].x, hr[p].y, hr[p].z, hr[p].w}, dw[4] = {dhr[p].x, dhr[p].y, dhr[p].z, dhr[p].w};
            float dot = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                dot += bf2f(hw[q] & 0xffffu) * bf2f(dw[q] & 0xffffu) + bf2f(hw[q] >> 16) * bf2f(dw[q] >> 16);
            // the 16 pieces of state row r are the 16 lanes of one DPP row
            dot = row16_allreduce(dot);
            if ((tid & 15) == 0) {
                sHdot[r] = dot;
                if constexpr (DEC) vgd[VGD_HD + r] = dot;
            }
        }
        auto f = [](uint32_t x) { return __uint_as_float(x); };
#pragma unroll
        for (int p = 0; p < NPER; ++p) {
            const int pc = tid + p * NTB, r = pc / (D / 8), c8 = (pc - r * (D / 8)) * 8;
            uint4 h, lo;
            const uint4 a0 = dl[2 * p], a1 = dl[2 * p + 1];
            pk2(f(a0.x), f(a0.y), h.x, lo.x);
            pk2(f(a0.z), f(a0.w), h.y, lo.y);
            pk2(f(a1.x), f(a1.y), h.z, lo.z);
            pk2(f(a1.z), f(a1.w), h.w, lo.w);
            *reinterpret_cast<uint4 *>(T16(VO_DLH) + r * LA + c8) = h;
            *reinterpret_cast<uint4 *>(T16(VO_DLL) + r * LA + c8) = lo;
            const uint4 t0v = td[2 * p], t1v = td[2 * p + 1];
            const float tv[8] = {f(t0v.x), f(t0v.y), f(t0v.z), f(t0v.w), f(t1v.x), f(t1v.y), f(t1v.z), f(t1v.w)};
            *reinterpret_cast<uint4 *>(T16(VO_TD) + r * LA + c8) =
                make_uint4(pk(tv[0], tv[1]), pk(tv[2], tv[3]), pk(tv[4], tv[5]), pk(tv[6], tv[7]));
            uint4 yv;
            if constexpr (DYF32) {
                const uint4 y0 = yr[2 * p], y1 = yr[2 * p + 1];
                yv = make_uint4(pk(f(y0.x), f(y0.y)), pk(f(y0.z), f(y0.w)), pk(f(y1.x), f(y1.y)), pk(f(y1.z), f(y1.w)));
            } else {
                yv = yr[p];
            }
            *reinterpret_cast<uint4 *>(T16(VO_DY) + r * LA + c8) = yv;
            const uint32_t vw[4] = {vr[p].x, vr[p].y, vr[p].z, vr[p].w};
            float vt = 0.f, dvv[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                vt += bf2f(vw[q] & 0xffffu) * tv[2 * q] + bf2f(vw[q] >> 16) * tv[2 * q + 1];
                dvv[2 * q] = bt[p] * tv[2 * q];
                dvv[2 * q + 1] = bt[p] * tv[2 * q + 1];
            }
            vt = row16_allreduce(vt);
            if ((tid & 15) == 0) sVT[r] = vt;
            if (r < n) {
                const size_t o = v0 + (size_t)r * v_row + c8;
                if (a.grad_dt == DT_BF16) {
                    *reinterpret_cast<uint4 *>(static_cast<bfr *>(a.dv) + o) =
                        make_uint4(pk(dvv[0], dvv[1]), pk(dvv[2], dvv[3]), pk(dvv[4], dvv[5]), pk(dvv[6], dvv[7]));
                } else if (a.grad_dt == DT_F32) {
                    float *dvp = static_cast<float *>(a.dv) + o;
                    *reinterpret_cast<float4 *>(dvp) = make_float4(dvv[0], dvv[1], dvv[2], dvv[3]);
                    *reinterpret_cast<float4 *>(dvp + 4) = make_float4(dvv[4], dvv[5], dvv[6], dvv[7]);
                } else {
#pragma unroll
                    for (int q = 0; q < 8; ++q) store_from_f32(a.dv, o + q, dvv[q], a.grad_dt);
                }
            }
        }
    }
    __syncthreads();
    // ---- S1 products over the value index: X1 = dY h^T, Y2 = TdD h^T, X2 = Delta dh'^T (Delta split),
    // dp = dY Delta^T and dAr = TdD Delta^T (Delta split)
    f4 X1[4], Y2[4], X2[4], dp[2], dAr[2];
#pragma unroll
    for (int t = 0; t < 4; ++t) X1[t] = Y2[t] = X2[t] = zero4();
    dp[0] = dp[1] = dAr[0] = dAr[1] = zero4();
    {
        const bfr *const tY = T16(VO_DY), *const tT = T16(VO_TD), *const tH = T16(VO_H), *const tDH = T16(VO_DHH);
        const bfr *const tLh = T16(VO_DLH), *const tLl = T16(VO_DLL);
#pragma unroll 2
        for (int k0 = 0; k0 < D; k0 += 32) {
            const bf8 ay = frag(tY, LA, r0, k0, l), at = frag(tT, LA, r0, k0, l);
            const bf8 ah = frag(tLh, LA, r0, k0, l), al = frag(tLl, LA, r0, k0, l);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf8 hb = frag(tH, LA, 64 * ch + 16 * t, k0, l);
                X1[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ay, hb, X1[t], 0, 0, 0);
                Y2[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at, hb, Y2[t], 0, 0, 0);
                const bf8 db = frag(tDH, LA, 64 * ch + 16 * t, k0, l);
                X2[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, db, X2[t], 0, 0, 0);
                X2[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, db, X2[t], 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const bf8 xh = frag(tLh, LA, 32 * ch + 16 * t, k0, l), xl = frag(tLl, LA, 32 * ch + 16 * t, k0, l);
                dp[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ay, xh, dp[t], 0, 0, 0);
                dp[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ay, xl, dp[t], 0, 0, 0);
                dAr[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at, xh, dAr[t], 0, 0, 0);
                dAr[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at, xl, dAr[t], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // the S1 tiles are read: the arena takes the pair cotangents and the permuted K, Q, G
    float *const sDP = F32(VO_DP), *const sDA = F32(VO_DA), *const sDPt = F32(VO_DPT), *const sDAt = F32(VO_DAT);
    bfr *const sKp = T16(VO_K), *const sQp = T16(VO_Q);
    float *const sGp = F32(VO_G);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = r0 + 4 * lg + e, s2 = 32 * ch + 16 * t + li;
            const float pv = s2 <= r ? dp[t][e] : 0.f, av = s2 < r ? -dAr[t][e] : 0.f;
            sDP[r * LDC + s2] = pv;
            sDA[r * LDC + s2] = av;
            sDPt[s2 * LDC + r] = pv;
            sDAt[s2 * LDC + r] = av;
            if constexpr (DEC) {
                // the blocks ck_vg_dg reads: the diagonal ones and those with a whole block between row and column
                const int S = 2 * ch + t;
                if (S == R || R - S >= 2) {
                    vgd[VGD_DP + r * C + s2] = pv;
                    vgd[VGD_DA + r * C + s2] = av;
                }
            }
        }
    {
        constexpr int PPER = C * (D / 8) / NTB;
#pragma unroll
        for (int p = 0; p < PPER; ++p) {
            const int pc = tid + p * NTB, r = pc / (D / 8), j0 = (pc - r * (D / 8)) * 8;
            const size_t o = (size_t)min(r, n - 1) * qk_row + j0;
            const uint4 xk = *reinterpret_cast<const uint4 *>(ksrc + o), xq = *reinterpret_cast<const uint4 *>(qsrc + o);
            const uint4 kq[2] = {r < n ? xk : make_uint4(0u, 0u, 0u, 0u), r < n ? xq : make_uint4(0u, 0u, 0u, 0u)};
            float g8[8];
            ld8(a.w.Gv + (ci * C + r) * D + j0, g8);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int pj = r * VLP + pcol(j0 + i);
                const uint32_t wk = (i < 2 ? kq[0].x : i < 4 ? kq[0].y : i < 6 ? kq[0].z : kq[0].w);
                const uint32_t wq = (i < 2 ? kq[1].x : i < 4 ? kq[1].y : i < 6 ? kq[1].z : kq[1].w);
                sKp[pj] = (bfr)(i & 1 ? wk >> 16 : wk & 0xffffu);
                sQp[pj] = (bfr)(i & 1 ? wq >> 16 : wq & 0xffffu);
                sGp[r * VLGp + pcol(j0 + i)] = g8[i];
            }
        }
        if (tid < D) sGCp[pcol(tid)] = a.w.Gv[(ci * C + C - 1) * D + tid];
    }
    __syncthreads();
    // this lane's elements: rows r0 + 4 lg + e, columns 64 ch + 16 t + li (permuted: 64 ch + 4 li + t)
    const int pc0 = 64 * ch + 4 * li;
    float Gr[4][4], kv[4][4], qv[4][4], gc[4];
    {
        const float4 g4 = *reinterpret_cast<const float4 *>(sGCp + pc0);
        gc[0] = g4.x; gc[1] = g4.y; gc[2] = g4.z; gc[3] = g4.w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = r0 + 4 * lg + e;
            const float4 x = *reinterpret_cast<const float4 *>(sGp + r * VLGp + pc0);
            Gr[e][0] = x.x; Gr[e][1] = x.y; Gr[e][2] = x.z; Gr[e][3] = x.w;
            const uint2 kk = *reinterpret_cast<const uint2 *>(sKp + r * VLP + pc0);
            const uint2 qq = *reinterpret_cast<const uint2 *>(sQp + r * VLP + pc0);
            kv[e][0] = bf2f(kk.x & 0xffffu); kv[e][1] = bf2f(kk.x >> 16); kv[e][2] = bf2f(kk.y & 0xffffu); kv[e][3] = bf2f(kk.y >> 16);
            qv[e][0] = bf2f(qq.x & 0xffffu); qv[e][1] = bf2f(qq.x >> 16); qv[e][2] = bf2f(qq.y & 0xffffu); qv[e][3] = bf2f(qq.y >> 16);
        }
    }
    // ---- the terms through the entry state and the exit-state adjoint: dq = X1 exp(G) (in X1), dk+ =
    // -beta Y2 exp(G) (in Y2), dk- = X2 exp(G_C - G) (in X2); dbeta -= Kg . Y2; dG_C's Kd term sum_r K * dk-
    float bp[4] = {0.f, 0.f, 0.f, 0.f}, gp[4] = {0.f, 0.f, 0.f, 0.f};
    // decays: this block's boundary values of G per channel, and the block sums of rho0 and sig0
    float gbt[4], gb2[4], b0[4], b0p[4];
    if constexpr (DEC) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            gbt[t] = R ? sGp[(r0 - 1) * VLGp + pc0 + t] : 0.f;
            gb2[t] = sGp[(r0 + 15) * VLGp + pc0 + t];
            b0[t] = b0p[t] = 0.f;
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float be = sB[r0 + 4 * lg + e];
        float rv[4], sv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float eG = ex2(Gr[e][t]), eD = ex2(gc[t] - Gr[e][t]);
            if constexpr (DEC) {
                const float rho0 = qv[e][t] * X1[t][e] - be * kv[e][t] * Y2[t][e], sig0 = kv[e][t] * X2[t][e];
                rv[t] = ex2(gbt[t]) * rho0;
                sv[t] = ex2(gc[t] - gb2[t]) * sig0;
                b0[t] = fmaf(ex2(Gr[e][t] - gbt[t]), rho0, b0[t]);
                b0p[t] = fmaf(ex2(gb2[t] - Gr[e][t]), sig0, b0p[t]);
            }
            bp[e] -= kv[e][t] * eG * Y2[t][e];
            X1[t][e] *= eG;
            Y2[t][e] *= -be * eG;
            X2[t][e] *= eD;
            gp[t] += kv[e][t] * X2[t][e];
        }
        if constexpr (DEC) {
            // the lane's four channels, in the permuted column order of the vgd tiles; the row and column roles add
            // rho1 and sig1 to these (the same lane reads back what it wrote)
            const int o = (r0 + 4 * lg + e) * D + pc0;
            *reinterpret_cast<float4 *>(vgd + VGD_RHO + o) = make_float4(rv[0], rv[1], rv[2], rv[3]);
            *reinterpret_cast<float4 *>(vgd + VGD_SIG + o) = make_float4(sv[0], sv[1], sv[2], sv[3]);
        }
    }
    if constexpr (DEC) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float x = b0[t], y = b0p[t];
            x += lane_xor16(x);
            x += lane_xor32(x);
            y += lane_xor16(y);
            y += lane_xor32(y);
            b0[t] = x;
            b0p[t] = y;
        }
        if (lg == 0) {
            *reinterpret_cast<float4 *>(vgd + VGD_B0 + R * D + pc0) = make_float4(b0[0], b0[1], b0[2], b0[3]);
            *reinterpret_cast<float4 *>(vgd + VGD_B0P + R * D + pc0) = make_float4(b0p[0], b0p[1], b0p[2], b0p[3]);
        }
    }
    f4 Z[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) Z[t] = zero4();
    // ---- pair terms below the diagonal blocks, row role of block R (contraction over the tokens s < 16 R, through
    // token bt = 16 R - 1): dq += (dP Y) exp(G_R - G_bt), Z += (dA Y) exp(G_R - G_bt), Y_sj = k_sj exp(G_bt - G_s)
    if (R >= 1) {
        const int bt = 16 * R - 1;
        f4 aq[4], az[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) aq[t] = az[t] = zero4();
        for (int k0 = 0; k0 < 16 * R; k0 += 32) {
            const int s0 = k0 + 8 * lg, rw = r0 + li;
            float xp[8], xa[8];
            ld8(sDP + rw * LDC + s0, xp);
            ld8(sDA + rw * LDC + s0, xa);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const bool ok = s0 + i < 16 * R;
                xp[i] = ok ? xp[i] : 0.f;
                xa[i] = ok ? xa[i] : 0.f;
            }
            bf8 ph, pl, zh, zl;
            split8(xp, ph, pl);
            split8(xa, zh, zl);
            // the factors of this lane's four columns (contiguous in the permuted tiles), one token at a time
            float y4[4][8];
            {
                const float4 gb4 = *reinterpret_cast<const float4 *>(sGp + bt * VLGp + pc0);
                const float gb[4] = {gb4.x, gb4.y, gb4.z, gb4.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int s2 = min(s0 + i, C - 1);
                    const bool ok = s0 + i < 16 * R;
                    const float4 g4 = *reinterpret_cast<const float4 *>(sGp + s2 * VLGp + pc0);
                    const uint2 kk = *reinterpret_cast<const uint2 *>(sKp + s2 * VLP + pc0);
                    const float gs4[4] = {g4.x, g4.y, g4.z, g4.w};
                    const float ks4[4] = {bf2f(kk.x & 0xffffu), bf2f(kk.x >> 16), bf2f(kk.y & 0xffffu), bf2f(kk.y >> 16)};
#pragma unroll
                    for (int t = 0; t < 4; ++t) y4[t][i] = ok ? ks4[t] * ex2(gb[t] - gs4[t]) : 0.f;
                }
            }
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                bf8 yh, yl;
                split8(y4[t], yh, yl);
                aq[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, yh, aq[t], 0, 0, 0);
                aq[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, yh, aq[t], 0, 0, 0);
                aq[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, yl, aq[t], 0, 0, 0);
                az[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(zh, yh, az[t], 0, 0, 0);
                az[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(zl, yh, az[t], 0, 0, 0);
                az[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(zh, yl, az[t], 0, 0, 0);
            }
        }
        if constexpr (DEC) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float be = sB[r0 + 4 * lg + e];
                float4 *const p4 = reinterpret_cast<float4 *>(vgd + VGD_RHO + (r0 + 4 * lg + e) * D + pc0);
                float4 x = *p4;
                x.x += qv[e][0] * aq[0][e] + be * kv[e][0] * az[0][e];
                x.y += qv[e][1] * aq[1][e] + be * kv[e][1] * az[1][e];
                x.z += qv[e][2] * aq[2][e] + be * kv[e][2] * az[2][e];
                x.w += qv[e][3] * aq[3][e] + be * kv[e][3] * az[3][e];
                *p4 = x;
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float gb = sGp[bt * VLGp + pc0 + t];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float eL = ex2(Gr[e][t] - gb);
                X1[t][e] += aq[t][e] * eL;
                Z[t][e] = az[t][e] * eL;
            }
        }
    }
    // ---- column role of block S = R (contraction over the tokens r > 16 S + 15, through that token b2):
    // dk- += (dP^T Xq + (diag(beta) dA)^T Xk) exp(G_b2 - G_S), X_rj = x_rj exp(G_r - G_b2)
    if (R <= 2) {
        const int b2 = 16 * R + 15, base = b2 + 1, cnt = C - base;
        f4 am[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) am[t] = zero4();
        for (int k0 = 0; k0 < cnt; k0 += 32) {
            const int q0 = base + k0 + 8 * lg, sw = r0 + li;
            float xp[8], xa[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int rq = min(q0 + i, C - 1);
                const bool ok = q0 + i < C;
                xp[i] = ok ? sDPt[sw * LDC + rq] : 0.f;
                xa[i] = ok ? sDAt[sw * LDC + rq] * sB[rq] : 0.f;
            }
            bf8 ph, pl, zh, zl;
            split8(xp, ph, pl);
            split8(xa, zh, zl);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int pj = 64 * ch + 4 * li + t;
                const float gb = sGp[b2 * VLGp + pj];
                float yq[8], yk[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int rq = min(q0 + i, C - 1);
                    const float ef = q0 + i < C ? ex2(sGp[rq * VLGp + pj] - gb) : 0.f;
                    yq[i] = bf2f(sQp[rq * VLP + pj]) * ef;
                    yk[i] = bf2f(sKp[rq * VLP + pj]) * ef;
                }
                bf8 qh, ql, kh, kl;
                split8(yq, qh, ql);
                split8(yk, kh, kl);
                am[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, qh, am[t], 0, 0, 0);
                am[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl, qh, am[t], 0, 0, 0);
                am[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph, ql, am[t], 0, 0, 0);
                am[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(zh, kh, am[t], 0, 0, 0);
                am[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(zl, kh, am[t], 0, 0, 0);
                am[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(zh, kl, am[t], 0, 0, 0);
            }
        }
        if constexpr (DEC) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float4 *const p4 = reinterpret_cast<float4 *>(vgd + VGD_SIG + (r0 + 4 * lg + e) * D + pc0);
                float4 x = *p4;
                x.x += kv[e][0] * am[0][e];
                x.y += kv[e][1] * am[1][e];
                x.z += kv[e][2] * am[2][e];
                x.w += kv[e][3] * am[3][e];
                *p4 = x;
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float gb = sGp[b2 * VLGp + pc0 + t];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                X2[t][e] += am[t][e] * ex2(gb - Gr[e][t]);
            }
        }
    }
    // ---- the diagonal block R, elementwise, along running products of the decays E_rs = prod_{s<u<=r} d_u (four
    // exponentials per step, d_u = 2^(G_u - G_{u-1}) of this lane's four channels).  Row role, s from the block's last
    // row down: dq_r += sum_{s <= r} dP_rs k_s E_rs, Z_r += sum_{s < r} dA_rs k_s E_rs.  Column role (this lane's
    // rows as s), r upwards: dk-_s += sum_{r >= s} (dP_rs q_r + beta_r dA_rs k_r) E_rs.  E is zero until the step
    // that reaches the lane's row.
    {
        float E[4][4], gn[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int t = 0; t < 4; ++t) E[e][t] = 0.f;
        {
            const float4 g4 = *reinterpret_cast<const float4 *>(sGp + (r0 + 15) * VLGp + pc0);
            gn[0] = g4.x; gn[1] = g4.y; gn[2] = g4.z; gn[3] = g4.w;
        }
        for (int sl = 15; sl >= 0; --sl) {
            const int s2 = r0 + sl;
            const float4 pv = *reinterpret_cast<const float4 *>(sDPt + s2 * LDC + r0 + 4 * lg);
            const float4 av = *reinterpret_cast<const float4 *>(sDAt + s2 * LDC + r0 + 4 * lg);
            const float4 g4 = *reinterpret_cast<const float4 *>(sGp + s2 * VLGp + pc0);
            const uint2 kk = *reinterpret_cast<const uint2 *>(sKp + s2 * VLP + pc0);
            const float pe[4] = {pv.x, pv.y, pv.z, pv.w}, ae[4] = {av.x, av.y, av.z, av.w};
            const float gs4[4] = {g4.x, g4.y, g4.z, g4.w};
            const float ks4[4] = {bf2f(kk.x & 0xffffu), bf2f(kk.x >> 16), bf2f(kk.y & 0xffffu), bf2f(kk.y >> 16)};
            float dn[4];  // the decay of token s + 1
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                dn[t] = ex2(gn[t] - gs4[t]);
                gn[t] = gs4[t];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // E is zero before this lane's row and becomes 1 on it: E d + [s == r] is exact in both cases
                const float at = sl == 4 * lg + e ? 1.f : 0.f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    E[e][t] = fmaf(E[e][t], dn[t], at);
                    const float kE = ks4[t] * E[e][t];
                    X1[t][e] = fmaf(pe[e], kE, X1[t][e]);
                    Z[t][e] = fmaf(ae[e], kE, Z[t][e]);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int t = 0; t < 4; ++t) E[e][t] = 0.f;
        {
            const float4 g4 = *reinterpret_cast<const float4 *>(sGp + r0 * VLGp + pc0);
            gn[0] = g4.x; gn[1] = g4.y; gn[2] = g4.z; gn[3] = g4.w;
        }
        for (int rl = 0; rl < 16; ++rl) {
            const int rq = r0 + rl;
            const float4 pv = *reinterpret_cast<const float4 *>(sDP + rq * LDC + r0 + 4 * lg);
            const float4 av = *reinterpret_cast<const float4 *>(sDA + rq * LDC + r0 + 4 * lg);
            const float4 g4 = *reinterpret_cast<const float4 *>(sGp + rq * VLGp + pc0);
            const uint2 kk = *reinterpret_cast<const uint2 *>(sKp + rq * VLP + pc0);
            const uint2 qq = *reinterpret_cast<const uint2 *>(sQp + rq * VLP + pc0);
            const float br = sB[rq];
            const float pe[4] = {pv.x, pv.y, pv.z, pv.w}, ae[4] = {av.x * br, av.y * br, av.z * br, av.w * br};
            const float gr4[4] = {g4.x, g4.y, g4.z, g4.w};
            const float kr4[4] = {bf2f(kk.x & 0xffffu), bf2f(kk.x >> 16), bf2f(kk.y & 0xffffu), bf2f(kk.y >> 16)};
            const float qr4[4] = {bf2f(qq.x & 0xffffu), bf2f(qq.x >> 16), bf2f(qq.y & 0xffffu), bf2f(qq.y >> 16)};
            float dr[4];  // the decay of token r
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                dr[t] = ex2(gr4[t] - gn[t]);
                gn[t] = gr4[t];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float at = rl == 4 * lg + e ? 1.f : 0.f;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    E[e][t] = fmaf(E[e][t], dr[t], at);
                    X2[t][e] = fmaf(fmaf(ae[e], kr4[t], pe[e] * qr4[t]), E[e][t], X2[t][e]);
                }
            }
        }
    }
    // ---- dk+ += diag(beta) Z, dbeta += k . Z; dG = q dq + k (dk+ - dk-)
    float dGv[4][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float be = sB[r0 + 4 * lg + e];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            bp[e] += kv[e][t] * Z[t][e];
            Y2[t][e] += be * Z[t][e];
            dGv[e][t] = qv[e][t] * X1[t][e] + kv[e][t] * (Y2[t][e] - X2[t][e]);
        }
    }
    __syncthreads();  // the transposed pair tiles are read: dG takes their space
    float *const sDG = F32(VO_DG);
    if constexpr (!DEC) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int t = 0; t < 4; ++t) sDG[(r0 + 4 * lg + e) * VLGp + 64 * ch + 16 * t + li] = dGv[e][t];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float rb = row16_allreduce(bp[e]);
        if (li == 0) sRow[ch][r0 + 4 * lg + e] = rb;
    }
    if constexpr (!DEC) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float x = gp[t];
            x += lane_xor16(x);
            x += lane_xor32(x);
            if (lg == 0) sDgc[R][64 * ch + 16 * t + li] = x;
        }
    }
    __syncthreads();
    // dg_log_u = sum_{r >= u} dG_r + dG_C (every token's log decay adds to G_C), in place: thread (segment gs of 16
    // rows, channel j) sums its segment, then adds the later segments' totals and dG_C while it writes the suffix sums
    if constexpr (!DEC) {
        const int j = tid & (D - 1), gs = tid >> 7;
        float tot = 0.f;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) tot += sDG[(16 * gs + rr) * VLGp + j];
        sSegT[gs][j] = tot;
        const float dgc = sDgc[0][j] + sDgc[1][j] + sDgc[2][j] + sDgc[3][j] + ex2(sGCp[pcol(j)]) * sHdot[j];
        __syncthreads();
        float run = dgc;
        for (int s3 = gs + 1; s3 < 4; ++s3) run += sSegT[s3][j];
#pragma unroll
        for (int rr = 15; rr >= 0; --rr) {
            const int r = 16 * gs + rr;
            run += sDG[r * VLGp + j];
            sDG[r * VLGp + j] = run;
        }
    }
    if (tid < C) {
        const int r = tid;
        if (r < n) a.dbeta[((size_t)b * a.Ts + t0 + r) * a.Hv + hv] = sVT[r] + sRow[0][r] + sRow[1][r];
    }
    if constexpr (!DEC) {
        __syncthreads();
        // d/d(log decay), coalesced over the channels
        constexpr int GPER = C * D / NTB;
        static_assert(GPER * NTB == C * D, "even split");
#pragma unroll
        for (int p = 0; p < GPER; ++p) {
            const int i = tid + p * NTB, r = i / D, j = i - r * D;
            if (r < n) a.dg[(((size_t)b * a.Ts + t0 + r) * a.Hv + hv) * D + j] = sDG[r * VLGp + j];
        }
    }
    // ---- dq | dk: this value head's parts summed over the key head's value heads.  They leave through an fp32
    // staging tile [64][dq 128 | dk 128] over the permuted K, Q, G tiles (dead since the diagonal loops), so that
    // each thread moves 8-element row pieces: the running sum (part rows, the same [dq | dk] layout) is read and
    // written, or the gradient stored, 16 bytes at a time.  A thread takes the same pieces for every value head and
    // reads back only what it wrote itself.
    {
        constexpr int LSQ = 2 * D + 4;
        static_assert(VO_K + C * LSQ * 4 <= VARENA && VO_K >= VO_DG + C * VLGp * 4, "dq | dk staging fits, clear of dG");
        float *const sQK = F32(VO_K);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int r = r0 + 4 * lg + e, j = 64 * ch + 16 * t + li;
                sQK[r * LSQ + j] = X1[t][e];
                sQK[r * LSQ + D + j] = Y2[t][e] + X2[t][e];
            }
        __syncthreads();
        constexpr int QPER = C * (2 * D / 8) / NTB;
        static_assert(QPER * NTB == C * (2 * D / 8), "even split");
#pragma unroll
        for (int p = 0; p < QPER; ++p) {
            const int pc = tid + p * NTB, r = pc / (2 * D / 8), c8 = (pc - r * (2 * D / 8)) * 8;
            if (r >= n) continue;
            float v[8];
            {
                const float4 x0 = *reinterpret_cast<const float4 *>(sQK + r * LSQ + c8);
                const float4 x1 = *reinterpret_cast<const float4 *>(sQK + r * LSQ + c8 + 4);
                v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w; v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
            }
            float *pr = part_row + (size_t)r * part_rs + c8;
            if (!first) {
                const float4 y0 = *reinterpret_cast<const float4 *>(pr), y1 = *reinterpret_cast<const float4 *>(pr + 4);
                v[0] += y0.x; v[1] += y0.y; v[2] += y0.z; v[3] += y0.w;
                v[4] += y1.x; v[5] += y1.y; v[6] += y1.z; v[7] += y1.w;
            }
            if (!last) {
                *reinterpret_cast<float4 *>(pr) = make_float4(v[0], v[1], v[2], v[3]);
                *reinterpret_cast<float4 *>(pr + 4) = make_float4(v[4], v[5], v[6], v[7]);
            } else {
                void *dst = c8 < D ? a.dq : a.dk;
                const size_t o = qk_out + (size_t)r * a.Hk * D + (c8 & (D - 1));
                if (a.grad_dt == DT_BF16) {
                    *reinterpret_cast<uint4 *>(static_cast<bfr *>(dst) + o) =
                        make_uint4(pk(v[0], v[1]), pk(v[2], v[3]), pk(v[4], v[5]), pk(v[6], v[7]));
                } else if (a.grad_dt == DT_F32) {
                    float *dp4 = static_cast<float *>(dst) + o;
                    *reinterpret_cast<float4 *>(dp4) = make_float4(v[0], v[1], v[2], v[3]);
                    *reinterpret_cast<float4 *>(dp4 + 4) = make_float4(v[4], v[5], v[6], v[7]);
                } else {
#pragma unroll
                    for (int q = 0; q < 8; ++q) store_from_f32(dst, o + q, v[q], a.grad_dt);
                }
            }
        }
    }
    __syncthreads();  // the arena is reused by the next value head
}

template <bool DYF32, bool DEC>
__global__ __launch_bounds__(NTB) void ck_bwd_local_vg_kernel(Args a) {
    typedef const __attribute__((address_space(4))) Args *KArgs;
    const int rep = a.Hv / a.Hk;
    for (int rr = 0; rr < rep; ++rr) {
        // the arguments are read anew for each value head instead of being held in scalar registers across it
        KArgs ap = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
        asm volatile("" : "+s"(ap));
        bwd_local_vg_head<DYF32, DEC>(*(const Args *)ap, blockIdx.x, blockIdx.y, blockIdx.z, rr, rep);
    }
}

// ---------------------------------------------------------------------------------------------- ck_vg_dg
//
// d/d(decay) of per-channel decays (the vector dg of tools/gdn_vjp.py:311-314, for the decay S * d of :174-179),
// two workgroups per (chunk, value head), each for 64 channels: thread (block
// U = its wave, channel j) for the 16 tokens u of block U (rows a..b2, bt = a - 1, G_-1 = 0, G the cumulative log
// decay of the chunk).
// Every term of d/d(log decay)_u is a pair term whose span s' < u <= r straddles u and which carries the factor
// exp(G_r - G_s'); d/d(decay)_u is that sum divided by d_u, and exp(G_r - G_s') / d_u = exp(G_r - G_u)
// exp(G_{u-1} - G_s'), two factors <= 1.  Grouped by where r and s' lie:
//   X_u = L_u Srow_u + R_u Scol_u + L_u R_u K_U + D4_u,  L_u = exp(G_{u-1} - G_bt),  R_u = exp(G_b2 - G_u)
//   Srow_u = sum_{r in U, r >= u} exp(G_r - G_u) RHO_r,  RHO = exp(G_bt) rho0 + rho1  (s' before the block)
//   Scol_u = sum_{s in U, s < u} exp(G_{u-1} - G_s) SIG_s,  SIG = exp(G_C - G_b2) sig0 + sig1  (r after it)
//   K_U = M_U + exp(G_bt) T0 + exp(G_C - G_b2) T0' + exp(G_bt + G_C - G_b2) <dh', h>  (both outside)
//   D4_u = sum_{r in U, r >= u} sum_{s in U, s < u} exp(G_r - G_u) exp(G_{u-1} - G_s) e'_rs  (both inside)
// with e'_rs = dP_rs q_r k_s + beta_r dA_rs k_r k_s, T0 = sum_{r > b2} exp(G_r - G_b2) rho0_r and T0' =
// sum_{s <= bt} exp(G_bt - G_s) sig0_s from the block sums B0_R = sum_{r in R} exp(G_r - G_bt(R)) rho0_r and
// B0'_S = sum_{s in S} exp(G_b2(S) - G_s) sig0_s, and M_U = sum_{r > b2, s <= bt} exp(G_r - G_b2) exp(G_bt - G_s)
// e'_rs from the transfers Q_RS = sum_{r in R, s in S} exp(G_r - G_bt(R)) exp(G_b2(S) - G_s) e'_rs of the block
// pairs (2, 0), (3, 0), (3, 1), which threads of blocks 0, 3 and 1 form.  Srow and Scol are scans along the block
// (S_u = RHO_u + d_{u+1} S_{u+1}; Scol_{u+1} = d_u Scol_u + SIG_u), L and R running products of the decays, and D4
// runs row by row (below).  Decays below 2^-64 count as 2^-64 (the cumulative log decays are formed that way).
constexpr int VDW = 64, NTV = 4 * VDW;  // channels per workgroup (two workgroups per chunk-head), threads

__global__ __launch_bounds__(NTV) void ck_vg_dg_kernel(Args a) {
    constexpr int LP = C + 4;  // 16-byte rows
    __shared__ __align__(16) float sP[C][LP], sA[C][LP];
    __shared__ float sBt[C];
    __shared__ float sQ[4][VDW];
    const int c = blockIdx.x >> 1, hv = blockIdx.y, b = blockIdx.z;
    const int hk = hv / (a.Hv / a.Hk);
    const int t0 = c * C, n = min(C, a.T - t0);
    const size_t ci = chunk_index(a, b, hv, c);
    const float *const vgd = a.w.vgd + ci * VGD_FLOATS;
    const float *const Gc = a.w.Gv + ci * C * D;  // log2 units
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    // the block index is uniform over a wave: row offsets stay in scalar registers and every load is a scalar base
    // plus the channel
    const int U = __builtin_amdgcn_readfirstlane(tid / VDW), a0 = 16 * U;
    const int jl = tid & (VDW - 1);
    const unsigned j = (blockIdx.x & 1) * VDW + jl;
    const size_t qk0 = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const bfr *const qsrc = static_cast<const bfr *>(a.q) + qk0, *const ksrc = static_cast<const bfr *>(a.k) + qk0;
    // row r of a [C][D] fp32 tile of this chunk-head, at this channel; tile_p: of the vgd tiles, whose columns are
    // in the permuted order of ck_bwd_local_vg's lanes (pcol)
    auto tile = [&](const float *base, int r) { return (base + (size_t)r * D)[j]; };
    const unsigned jp = pcol(j);
    auto tile_p = [&](const float *base, int r) { return (base + (size_t)r * D)[jp]; };
    // q or k of row r of this channel, zero past the sequence
    auto ld_qk = [&](const bfr *src, int r) {
        const float x = bf2f((src + (size_t)min(r, n - 1) * qk_row)[j]);
        return r < n ? x : 0.f;
    };
    // the blocks of dP and dA in use: (0,0) (1,1) (2,2) (3,3) (2,0) (3,0) (3,1)
    for (int i = tid; i < 7 * 256; i += NTV) {
        const int blk = i >> 8, e = i & 255;
        const int R = blk < 4 ? blk : blk == 6 ? 3 : blk - 2, S = blk < 4 ? blk : blk == 6 ? 1 : 0;
        const int r = 16 * R + (e >> 4), s = 16 * S + (e & 15);
        sP[r][s] = vgd[VGD_DP + r * C + s];
        sA[r][s] = vgd[VGD_DA + r * C + s];
    }
    if (tid < C) {
        const float xb = a.beta[((size_t)b * a.Ts + t0 + min(tid, n - 1)) * a.Hv + hv];
        sBt[tid] = tid < n ? xb : 0.f;
    }
    // G at the last row of each block; this block's rows and decays d_i = 2^(G_i - G_{i-1})
    float gB[4], G[16], d[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) gB[i] = tile(Gc, 16 * i + 15);
#pragma unroll
    for (int i = 0; i < 16; ++i) G[i] = tile(Gc, a0 + i);
    const float gbt = U == 0 ? 0.f : U == 1 ? gB[0] : U == 2 ? gB[1] : gB[2];
    const float gb2 = U == 0 ? gB[0] : U == 1 ? gB[1] : U == 2 ? gB[2] : gB[3];
    const float gC = gB[3];
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i] = ex2(G[i] - (i ? G[i - 1] : gbt));
    float qv[16], kv[16], B0[4], B0P[4];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        qv[i] = ld_qk(qsrc, a0 + i);
        kv[i] = ld_qk(ksrc, a0 + i);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        B0[i] = tile_p(vgd + VGD_B0, i);
        B0P[i] = tile_p(vgd + VGD_B0P, i);
    }
    // X = L Srow + R Scol (the K term waits for the transfers)
    float X[16];
    {
        float RHO[16], SIG[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            RHO[i] = tile_p(vgd + VGD_RHO, a0 + i);
            SIG[i] = tile_p(vgd + VGD_SIG, a0 + i);
        }
        // Srow (a scan from the block's end) times L_i = exp(G_{i-1} - G_bt), then R_i Scol_i with R_i = exp(G_b2 -
        // G_i); L and R as running products of the decays
        float S = 0.f;
#pragma unroll
        for (int i = 15; i >= 0; --i) {
            S = i < 15 ? fmaf(d[i + 1], S, RHO[i]) : RHO[i];
            X[i] = S;
        }
        float L = 1.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            X[i] *= L;
            L *= d[i];
        }
        float rr[16], Rf = 1.f;
#pragma unroll
        for (int i = 15; i >= 0; --i) {
            rr[i] = Rf;
            Rf *= d[i];
        }
        float Sc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            X[i] = fmaf(rr[i], Sc, X[i]);
            Sc = fmaf(d[i], Sc, SIG[i]);
        }
    }
    const float hdot = (vgd + VGD_HD)[j];
    __syncthreads();  // dP, dA, beta
    // the transfer of block pair (R, S): threads of block 0 take (2, 0), of block 3 (3, 0), of block 1 (3, 1)
    if (U != 2) {
        const int R = U == 0 ? 2 : 3, S = U == 1 ? 1 : 0;
        const float gtR = R == 2 ? gB[1] : gB[2], gbS = S == 0 ? gB[0] : gB[1];
        float kap[16], qr[16], kr[16], er[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int s = 16 * S + i, r = 16 * R + i;
            kap[i] = ld_qk(ksrc, s) * ex2(gbS - tile(Gc, s));
            qr[i] = ld_qk(qsrc, r);
            kr[i] = ld_qk(ksrc, r) * sBt[r];
            er[i] = ex2(tile(Gc, r) - gtR);
        }
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 16 * R + i;
            float pp = 0.f, pa = 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                pp = fmaf(sP[r][16 * S + e], kap[e], pp);
                pa = fmaf(sA[r][16 * S + e], kap[e], pa);
            }
            acc = fmaf(er[i], fmaf(qr[i], pp, kr[i] * pa), acc);
        }
        sQ[U][jl] = acc;
    }
    __syncthreads();  // transfers
    {
        float T0 = 0.f, T0p = 0.f;
#pragma unroll
        for (int R = 1; R < 4; ++R)
            if (R > U) T0 = fmaf(ex2(gB[R - 1] - gb2), B0[R], T0);
#pragma unroll
        for (int S = 0; S < 3; ++S)
            if (S < U) T0p = fmaf(ex2(gbt - gB[S]), B0P[S], T0p);
        const float M = U == 1 ? sQ[0][jl] + ex2(gB[2] - gB[1]) * sQ[3][jl]
                        : U == 2 ? ex2(gB[1] - gB[0]) * sQ[3][jl] + sQ[1][jl] : 0.f;
        const float K = M + ex2(gbt) * T0 + ex2(gC - gb2) * T0p + ex2(gbt + gC - gb2) * hdot;
        // L_i R_i = prod of the block's decays other than d_i
        float L = 1.f, rr[16], Rf = 1.f;
#pragma unroll
        for (int i = 15; i >= 0; --i) {
            rr[i] = Rf;
            Rf *= d[i];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            X[i] = fmaf(L * rr[i], K, X[i]);
            L *= d[i];
        }
    }
    // D4, one row r of the block at a time: cs[u] = c_r(u) = sum_{s in U, s < u} exp(G_{u-1} - G_s) e'_rs
    // (c_r(u + 1) = d_u c_r(u) + e'_ru), then X_u += exp(G_r - G_u) c_r(u) for u <= r, the factor a running product
    // from u = r down.  Each row's LDS reads go through an address that depends on the previous row's result: the
    // compiler would otherwise hoist the reads of every row to the start and spill.
    {
        float link = 0.f;
#pragma unroll
        for (int r = 1; r < 16; ++r) {
            int ro = (a0 + r) * LP + a0;
            asm volatile("" : "+v"(ro) : "v"(link));
            const float *const prow = &sP[0][0] + ro, *const arow = &sA[0][0] + ro;
            const float qr = qv[r], bkr = sBt[a0 + r] * kv[r];
            float cs[16];
            float cc = 0.f;
#pragma unroll
            for (int u = 0; u < r; ++u) {
                const float ep = kv[u] * fmaf(prow[u], qr, bkr * arow[u]);
                cc = fmaf(d[u], cc, ep);
                cs[u + 1] = cc;
            }
            float E = 1.f;
#pragma unroll
            for (int u = r; u >= 1; --u) {
                X[u] = fmaf(E, cs[u], X[u]);
                E *= d[u];
            }
            link = cc;
        }
    }
    // X is complete here: without this the compiler sinks the row updates into the conditional stores below and
    // keeps every term live until then
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(X[i]));
    float *const dgb = a.dg + (((size_t)b * a.Ts + t0 + a0) * a.Hv + hv) * D;
    const size_t drow = (size_t)a.Hv * D;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (a0 + i < n) (dgb + i * drow)[j] = X[i];
}

void launch_vg_local(const Args &a, hipStream_t st) {
    const bool dec = a.gate == GATE_DECAY_VEC;
    const dim3 grid(a.NC, a.Hk, a.B);
    if (a.dy_dt == DT_F32) {
        if (dec) hipLaunchKernelGGL((ck_bwd_local_vg_kernel<true, true>), grid, dim3(NTB), 0, st, a);
        else hipLaunchKernelGGL((ck_bwd_local_vg_kernel<true, false>), grid, dim3(NTB), 0, st, a);
    } else {
        if (dec) hipLaunchKernelGGL((ck_bwd_local_vg_kernel<false, true>), grid, dim3(NTB), 0, st, a);
        else hipLaunchKernelGGL((ck_bwd_local_vg_kernel<false, false>), grid, dim3(NTB), 0, st, a);
    }
}

void launch_vg_dg(const Args &a, hipStream_t st) {
    if (a.gate == GATE_DECAY_VEC) hipLaunchKernelGGL(ck_vg_dg_kernel, dim3(2 * a.NC, a.Hv, a.B), dim3(NTV), 0, st, a);
}

}  // namespace ck
}  // namespace gdn
