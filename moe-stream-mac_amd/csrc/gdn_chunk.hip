// Chunked (WY / UT) form of the Gated DeltaNet forward and VJP for gfx950, chunk C = 64, Dk = Dv = D = 128.
//
// Per chunk of one head with entry state h = S^T ([Dk][Dv]), log decays g, G_r = sum_{u<=r} g_u (fp64),
// gamma = exp(G), Gam_rs = exp(G_r - G_s) for s <= r:
//   A = strict_lower(diag(beta) (K K^T) * Gam),  T = (I + A)^-1,  W = T diag(beta gamma) K,  U = T diag(beta) V
//   Delta = U - W h,  P = lower(Q K^T * Gam),  Y = diag(gamma) Q h + P Delta,
//   h' = gamma_C h + K^T diag(gamma_C / gamma) Delta
// which equals the token recurrence of engine/include/gdn.h:27-38 / tools/gdn_vjp.py:3-6 exactly in exact
// arithmetic.  The reverse pass is the adjoint of these matrix expressions (chunk-parallel except for the
// state adjoint, which runs backward over chunks like the forward state does).
//
// Kernels (one set for fp32 inputs on v_mfma_f32_16x16x4_f32, one for bf16 inputs on v_mfma_f32_16x16x32_bf16;
// fp32 accumulation, the state stays fp32 in the accumulators):
//   ck_prep[_bf16]       grid (NC, Hv, B): G, T (blocked 16x16 unit-lower inverse), W, U, P of one chunk.
//   ck_fwd[_bf16]        grid (D/VS, Hv, B): sequential over chunks; one value slice of h lives in accumulators.
//   ck_bwd_seq[_bf16]    grid (D/VS, Hv, B): reverse over chunks; the state adjoint dh and dDelta.
//   ck_bwd_local[_bf16]  grid (NC, Hk, B): dv, dbeta, dg of one chunk for each value head of a key head in turn,
//                        and the key head's dq, dk (the value heads' parts summed in order).
#include "gdn_chunk_common.h"

namespace gdn {
namespace ck {

// ---------------------------------------------------------------------------------------------- ck_prep

// The element dtypes of a launch of the fp32 kernel set: constants when AF32 (inputs, cotangent, outputs and
// gradients all fp32), so that no load or store of a tile sits under a dtype branch (where the branches join, the
// compiler waits for every load in flight); read from the arguments otherwise (fp16 inputs).
#define DTYPES_OF(args)                                                                     \
    const int k_in_dt = AF32 ? (int)DT_F32 : (args).in_dt, k_dy_dt = AF32 ? (int)DT_F32 : (args).dy_dt, \
              k_out_dt = AF32 ? (int)DT_F32 : (args).out_dt, k_grad_dt = AF32 ? (int)DT_F32 : (args).grad_dt; \
    (void)k_in_dt; (void)k_dy_dt; (void)k_out_dt; (void)k_grad_dt

template <bool AF32>
__global__ __launch_bounds__(NTP) void ck_prep_kernel(Args a) {
    DTYPES_OF(a);
    __shared__ __align__(16) float sK[C * LD];
    __shared__ __align__(16) float sX[C * LD];
    __shared__ __align__(16) float sA[C * LDC];
    __shared__ __align__(16) float sT[C * LDC];
    __shared__ float scratch[3 * 256];
    __shared__ double sG[C];
    __shared__ float sB[C], sGam[C], sRc[C];

    const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk), t0 = c * C, n = min(C, T - t0);
    const size_t ci = chunk_index(a, b, hv, c);
    const size_t qk0 = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * a.Ts + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;

    TileRegs<C, D, NTP> rV;  // V is needed only after the inverse: fetch it now, store it later
    tile_fetch(rV, elem_ptr(a.v, v0, k_in_dt), v_row, n, k_in_dt);
    load_tile<C, D, NTP>(sK, LD, elem_ptr(a.k, qk0, k_in_dt), qk_row, n, k_in_dt);
    load_tile<C, D, NTP>(sX, LD, elem_ptr(a.q, qk0, k_in_dt), qk_row, n, k_in_dt);
    if (tid < C) {
        // inclusive prefix sum of the log decays in fp64 across wave 0
        float bt = 0.f, gl = 0.f;
        if (tid < n) {
            const size_t gi = ((size_t)b * a.Ts + t0 + tid) * a.Hv + hv;
            bt = a.beta[gi];
            gl = gate_log(a.g[gi], a.gate);
        }
        const double x = wave_prefix_sum((double)gl);
        sB[tid] = bt;
        sG[tid] = x;
        sGam[tid] = expf((float)x);
        sRc[tid] = expf((float)(readlane_f64(x, 63) - x));  // gamma_C / gamma_r
    }
    __syncthreads();
    // K K^T (waves 0-3) and Q K^T (waves 4-7): each wave a 16-row strip of 4 tiles
    {
        const int r0 = 16 * (w & 3);
        const bool isq = w >= 4;
        f4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = zero4();
        mma_strip<D, 4>(acc, (isq ? sX : sK) + r0 * LD, LD, 1, sK, 1, LD, 16 * LD);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = r0 + 4 * lg + e, s2 = 16 * t + li;
                const float gam = s2 <= r ? expf((float)(sG[r] - sG[s2])) : 0.f;
                if (isq) a.w.P[ci * C * C + r * C + s2] = acc[t][e] * gam;
                else sA[r * LDC + s2] = s2 < r ? sB[r] * acc[t][e] * gam : 0.f;
            }
    }
    __syncthreads();
    unit_lower_inverse<NTP>(sA, sT, scratch);
    for (int i = tid; i < C * D; i += NTP) {
        const int r = i / D, j = i - r * D;
        sK[r * LD + j] *= sB[r] * sGam[r];
    }
    {
        const float *bp = sB;
        tile_store(sX, LD, rV, k_in_dt, [bp](int r) { return bp[r]; });
    }
    __syncthreads();
    // W = T diag(beta gamma) K (waves 0-3) and U = T diag(beta) V (waves 4-7), 16-row strips of 8 tiles
    {
        const int r0 = 16 * (w & 3);
        const bool isu = w >= 4;
        f4 acc[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] = zero4();
        if (isu) mma_strip<C, 8>(acc, sT + r0 * LDC, LDC, 1, sX, LD, 1, 16);
        else mma_strip<C, 8>(acc, sT + r0 * LDC, LDC, 1, sK, LD, 1, 16);
        float *out = isu ? a.w.U : a.w.W;
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) out[ci * C * D + (r0 + 4 * lg + e) * D + 16 * t + li] = acc[t][e];
    }
    if (!a.fwd_only)
        for (int i = tid; i < C * C; i += NTP) a.w.T[ci * C * C + i] = sT[(i / C) * LDC + (i % C)];
    if (tid < C) a.w.G[ci * C + tid] = sG[tid];
}

// ---------------------------------------------------------------------------------------------- ck_fwd


// Row scalings read the chunk's cumulative log decays from LDS: gamma_r = exp(G_r), rc_r = exp(G_{C-1} - G_r).
struct GamScale {
    const double *G;
    __device__ float operator()(int r) const { return expf((float)G[r]); }
};
struct RcScale {
    const double *G;
    __device__ float operator()(int r) const { return expf((float)(G[C - 1] - G[r])); }
};

template <int VS, int MODE, bool AF32>
__global__ __launch_bounds__(NTS) void ck_fwd_kernel(Args a) {
    DTYPES_OF(a);
    constexpr bool kTiles = MODE != FWD_ONLY, kOut = MODE != FWD_RECOMPUTE;
    constexpr int LV = VS + 4;
    constexpr int NTN = VS / 16;                 // value tiles of the slice
    constexpr int DN = NTN >= 2 ? NTN / 2 : 1;   // value tiles per wave for [C][VS] products
    __shared__ __align__(16) float sW[C * LD];  // W, then P (stride LDC)
    __shared__ __align__(16) float sQ[C * LD];  // Q, then K diag(gamma_C / gamma)
    __shared__ __align__(16) float sU[C * LV];
    __shared__ __align__(16) float sH[D * LV];  // h slice, [j][i]
    __shared__ __align__(16) float sD[C * LV];  // Delta slice
    __shared__ double sG[C];

    const SeqBlock sb = seq_block();
    const SeqRange sr = seq_range<MODE>(a, sb.b);
    const int i0 = sb.slice * VS, hv = sb.hv, b = sr.b, cb = sr.cb, ce = sr.ce;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk);
    const size_t head = (size_t)b * a.Hv + hv;
    const size_t qk_row = (size_t)a.Hk * D;
    const int mrow = 16 * (w & 3);                              // rows of this wave's [C][VS] tiles
    const bool cwave = NTN >= 2 || w < 4;                       // waves that own [C][VS] tiles
    const int nt0 = NTN >= 2 ? (w >> 2) * DN : 0;               // first value tile of those

    f4 h[NTN];  // rows j = 16w.., value tiles 0..NTN-1
#pragma unroll
    for (int t = 0; t < NTN; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 16 * w + 4 * lg + e, i = i0 + 16 * t + li;
            h[t][e] = sr.s0 ? sr.s0[(head * D + i) * D + j] : 0.f;
        }
    TileRegs<C, D, NTS> rW, rQ, rK;
    TileRegs<C, VS, NTS> rU;
    TileRegs<C, C, NTS> rP;
    double rG = 0.0;
    auto fetchA = [&](int c) {
        const size_t ci = head * a.NC + c;
        const size_t qk0 = (((size_t)b * a.Ts + c * C) * a.Hk + hk) * D;
        const int n = min(C, T - c * C);
        tile_fetch(rW, a.w.W + ci * C * D, D, C, DT_F32);
        tile_fetch(rU, a.w.U + ci * C * D + i0, D, C, DT_F32);
        tile_fetch(rQ, elem_ptr(a.q, qk0, k_in_dt), qk_row, n, k_in_dt);
        if (tid < C) rG = a.w.G[ci * C + tid];
    };
    auto fetchB = [&](int c) {
        const size_t ci = head * a.NC + c;
        const size_t qk0 = (((size_t)b * a.Ts + c * C) * a.Hk + hk) * D;
        const int n = min(C, T - c * C);
        tile_fetch(rP, a.w.P + ci * C * C, C, C, DT_F32);
        tile_fetch(rK, elem_ptr(a.k, qk0, k_in_dt), qk_row, n, k_in_dt);
    };
    fetchA(cb);
    fetchB(cb);
    for (int c = cb; c < ce; ++c) {
        const int t0 = c * C, n = min(C, T - t0);
        const size_t ci = head * a.NC + c;
        if (float *sp = snap_at<MODE>(a, c)) store_state_acc<NTN>(sp, h, head, i0, w, lg, li);
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NTN; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) sH[(16 * w + 4 * lg + e) * LV + 16 * t + li] = h[t][e];
        tile_store(sW, LD, rW, DT_F32, NoScale{});
        tile_store(sU, LV, rU, DT_F32, NoScale{});
        tile_store(sQ, LD, rQ, k_in_dt, NoScale{});
        if (tid < C) sG[tid] = rG;
        __syncthreads();
        if (c + 1 < ce) fetchA(c + 1);
        if (kTiles) store_state_slice<VS, LV, NTS>(a.w.H + ci * D * D, sH, i0);
        // Delta = U - W h ; Yi = Q h
        f4 wh[DN], yi[DN];
#pragma unroll
        for (int t = 0; t < DN; ++t) wh[t] = yi[t] = zero4();
        if (cwave) {
            mma_strip<D, DN>(wh, sW + mrow * LD, LD, 1, sH + 16 * nt0, LV, 1, 16);
            mma_strip<D, DN>(yi, sQ + mrow * LD, LD, 1, sH + 16 * nt0, LV, 1, 16);
#pragma unroll
            for (int t = 0; t < DN; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = mrow + 4 * lg + e, ii = 16 * (nt0 + t) + li;
                    const float dl = sU[r * LV + ii] - wh[t][e];
                    sD[r * LV + ii] = dl;
                    if (kTiles) a.w.Dl[ci * C * D + r * D + i0 + ii] = dl;
                }
        }
        __syncthreads();
        tile_store(sW, LDC, rP, DT_F32, NoScale{});
        tile_store(sQ, LD, rK, k_in_dt, RcScale{sG});
        __syncthreads();
        if (c + 1 < ce) fetchB(c + 1);
        if (cwave && kOut) {
            // Y = diag(gamma) Q h + P Delta
#pragma unroll
            for (int t = 0; t < DN; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) yi[t][e] *= expf((float)sG[mrow + 4 * lg + e]);
            mma_strip<C, DN>(yi, sW + mrow * LDC, LDC, 1, sD + 16 * nt0, LV, 1, 16);
#pragma unroll
            for (int t = 0; t < DN; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = mrow + 4 * lg + e, ii = 16 * (nt0 + t) + li;
                    if (r < n)
                        store_from_f32(a.y, (((size_t)b * a.Ts + t0 + r) * a.Hv + hv) * D + i0 + ii, yi[t][e],
                                       k_out_dt);
                }
        }
        // h = gamma_C h + Ktilde^T Delta
        const float gC = expf((float)sG[C - 1]);
#pragma unroll
        for (int t = 0; t < NTN; ++t) h[t] *= gC;
        mma_strip<C, NTN>(h, sQ + 16 * w, 1, LD, sD, LV, 1, 16);
    }
    if (kOut && a.state_T) store_state_acc<NTN>(a.state_T, h, head, i0, w, lg, li);
}

// ---------------------------------------------------------------------------------------------- ck_bwd_seq

template <int VS, bool AF32>
__global__ __launch_bounds__(NTS) void ck_bwd_seq_kernel(Args a) {
    DTYPES_OF(a);
    constexpr int LV = VS + 4;
    constexpr int NTN = VS / 16;
    constexpr int DN = NTN >= 2 ? NTN / 2 : 1;
    __shared__ __align__(16) float sW[C * LD];   // P (stride LDC), then W
    __shared__ __align__(16) float sQ[C * LD];   // K, then Q
    __shared__ __align__(16) float sY[C * LV];   // dY slice
    __shared__ __align__(16) float sYg[C * LV];  // diag(gamma) dY slice
    // dh slice [j][i]; after the dDelta products (second barrier) T [r][s] (stride LDC) until the step ends
    __shared__ __align__(16) float sH[(D * LV > C * LDC) ? D * LV : C * LDC];
    __shared__ __align__(16) float sD[C * LV];   // dDelta slice
    __shared__ double sG[C];
    float *const sT = sH;

    const SeqBlock sb = seq_block();
    const int i0 = sb.slice * VS, hv = sb.hv, b = sb.b;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk);
    const size_t head = (size_t)b * a.Hv + hv;
    const size_t qk_row = (size_t)a.Hk * D, v_row = (size_t)a.Hv * D;
    const int mrow = 16 * (w & 3);
    const bool cwave = NTN >= 2 || w < 4;
    const int nt0 = NTN >= 2 ? (w >> 2) * DN : 0;

    f4 dh[NTN];
#pragma unroll
    for (int t = 0; t < NTN; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 16 * w + 4 * lg + e, i = i0 + 16 * t + li;
            dh[t][e] = a.dstate_T ? a.dstate_T[(head * D + i) * D + j] : 0.f;
        }
    TileRegs<C, C, NTS> rP, rT;
    TileRegs<C, D, NTS> rK, rW, rQ;
    TileRegs<C, VS, NTS> rY;
    double rG = 0.0;
    auto fetchA = [&](int c) {
        const size_t ci = head * a.NC + c;
        const size_t qk0 = (((size_t)b * a.Ts + c * C) * a.Hk + hk) * D;
        const size_t v0 = (((size_t)b * a.Ts + c * C) * a.Hv + hv) * D;
        const int n = min(C, T - c * C);
        tile_fetch(rP, a.w.P + ci * C * C, C, C, DT_F32);
        tile_fetch(rK, elem_ptr(a.k, qk0, k_in_dt), qk_row, n, k_in_dt);
        tile_fetch(rY, elem_ptr(a.dy, v0 + i0, k_dy_dt), v_row, n, k_dy_dt);
        if (tid < C) rG = a.w.G[ci * C + tid];
    };
    auto fetchB = [&](int c) {
        const size_t ci = head * a.NC + c;
        const size_t qk0 = (((size_t)b * a.Ts + c * C) * a.Hk + hk) * D;
        const int n = min(C, T - c * C);
        tile_fetch(rW, a.w.W + ci * C * D, D, C, DT_F32);
        tile_fetch(rQ, elem_ptr(a.q, qk0, k_in_dt), qk_row, n, k_in_dt);
        tile_fetch(rT, a.w.T + ci * C * C, C, C, DT_F32);
    };
    fetchA(a.NC - 1);
    fetchB(a.NC - 1);
    for (int c = a.NC - 1; c >= 0; --c) {
        const size_t ci = head * a.NC + c;
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NTN; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) sH[(16 * w + 4 * lg + e) * LV + 16 * t + li] = dh[t][e];
        tile_store(sW, LDC, rP, DT_F32, NoScale{});
        tile_store(sQ, LD, rK, k_in_dt, NoScale{});
        tile_store(sY, LV, rY, k_dy_dt, NoScale{});
        if (tid < C) sG[tid] = rG;
        __syncthreads();
        tile_store(sYg, LV, rY, k_dy_dt, GamScale{sG});   // before rY is refilled
        if (c > 0) fetchA(c - 1);
        store_state_slice<VS, LV, NTS>(a.w.dH + ci * D * D, sH, i0);
        // dDelta = diag(gamma_C / gamma) K dh' + P^T dY
        if (cwave) {
            f4 kd[DN], pd[DN];
#pragma unroll
            for (int t = 0; t < DN; ++t) kd[t] = pd[t] = zero4();
            mma_strip<D, DN>(kd, sQ + mrow * LD, LD, 1, sH + 16 * nt0, LV, 1, 16);
            mma_strip<C, DN>(pd, sW + mrow, 1, LDC, sY + 16 * nt0, LV, 1, 16);
#pragma unroll
            for (int t = 0; t < DN; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = mrow + 4 * lg + e, ii = 16 * (nt0 + t) + li;
                    sD[r * LV + ii] = kd[t][e] * expf((float)(sG[C - 1] - sG[r])) + pd[t][e];
                }
        }
        __syncthreads();
        tile_store(sW, LD, rW, DT_F32, NoScale{});
        tile_store(sQ, LD, rQ, k_in_dt, NoScale{});
        tile_store(sT, LDC, rT, DT_F32, NoScale{});  // over dh', read before the barrier above
        __syncthreads();
        if (c > 0) fetchB(c - 1);
        // saved TdD = T^T dDelta, the only form in which ck_bwd_local_kernel needs T and dDelta
        if (cwave) {
            f4 tdd[DN];
#pragma unroll
            for (int t = 0; t < DN; ++t) tdd[t] = zero4();
            mma_strip<C, DN>(tdd, sT + mrow, 1, LDC, sD + 16 * nt0, LV, 1, 16);
#pragma unroll
            for (int t = 0; t < DN; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    a.w.dDl[ci * C * D + (size_t)(mrow + 4 * lg + e) * D + i0 + 16 * (nt0 + t) + li] = tdd[t][e];
        }
        // dh = gamma_C dh' + Q^T diag(gamma) dY - W^T dDelta
        const float gC = expf((float)sG[C - 1]);
        f4 wd[NTN];
#pragma unroll
        for (int t = 0; t < NTN; ++t) {
            dh[t] *= gC;
            wd[t] = zero4();
        }
        mma_strip<C, NTN>(dh, sQ + 16 * w, 1, LD, sYg, LV, 1, 16);
        mma_strip<C, NTN>(wd, sW + 16 * w, 1, LD, sD, LV, 1, 16);
#pragma unroll
        for (int t = 0; t < NTN; ++t) dh[t] -= wd[t];
    }
    if (a.dstate0) {
#pragma unroll
        for (int t = 0; t < NTN; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 16 * w + 4 * lg + e, i = i0 + 16 * t + li;
                a.dstate0[(head * D + i) * D + j] = dh[t][e];
            }
    }
}

// ---------------------------------------------------------------------------------------------- ck_bwd_local


// dbeta and dg of one chunk from the pair terms, after the barrier that completes sE / sRow / sLast:
//   sE [C][LDC]      E[r][s'] (pair terms, s' < r); overwritten with row prefix sums
//   sRow[0..2][h][r] the two column halves' row sums of the boundary terms, the pairs (C-1, r) and dbeta
//   sLast[8]         the waves' parts of <dh', h> (times last_scale: the pair (C-1, chunk start))
//   sScan[2][C]      scratch
// dg_u = sum_{r >= u} (sum_{s' < u} E[r][s'] + Eb[r]) + sum_{s < u} T2[s]: row prefix sums in 8-lane segments,
// column sums in 8-lane groups, and the Eb suffix / T2 prefix as wave-0 DPP scans (the suffix as a prefix over
// lanes holding Eb in reverse row order).  Every thread takes part.
template <int NTH>
__device__ __forceinline__ void chunk_dg_dbeta(float *sE, const float (*sRow)[2][C], const float *sLast, float last_scale,
                                               float (*sScan)[C], const Args &a, int b, int hv, int t0, int n,
                                               int tid) {
    static_assert(NTH == C * 8, "eight threads per row / column");
    const size_t g0 = ((size_t)b * a.Ts + t0) * a.Hv + hv;
    static_assert(C == 64, "one wave scans the chunk");
    if (tid < C) {
        const int r = tid, rs = C - 1 - tid;  // rs: this lane's row of the suffix scan
        float eb = sRow[0][0][rs] + sRow[0][1][rs];
        if (rs == C - 1)
            for (int i = 0; i < 8; ++i) eb += sLast[i] * last_scale;
        const float t2 = r < C - 1 ? sRow[1][0][r] + sRow[1][1][r] : 0.f;  // pair (C-1, r)
        if (r < n) a.dbeta[g0 + (size_t)r * a.Hv] = sRow[2][0][r] + sRow[2][1][r];
        const float su = wave_prefix_sum(eb), pr = wave_prefix_sum(t2);
        // exclusive prefix by a one-lane shift, not by subtracting t2: every partial sum holds only terms whose span
        // straddles the token (no cancellation of larger terms)
        const float prx = wave_shr1(pr);
        sScan[0][rs] = su;                // sum_{r' >= rs} Eb[r']
        sScan[1][r] = r > 0 ? prx : 0.f;  // sum_{s < r} T2[s]
    }
    {
        // sE[r][s2] <- sum_{s' < s2, s' < r} E[r][s']
        const int r = tid >> 3, part = tid & 7, s0 = 8 * part;
        float *row = sE + r * LDC + s0;
        const float4 x0 = *reinterpret_cast<const float4 *>(row), x1 = *reinterpret_cast<const float4 *>(row + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float ex[8], run = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ex[i] = run;
            run += s0 + i < r ? xv[i] : 0.f;
        }
        // inclusive scan over the row's 8 parts (DPP row shifts; a shifted value from another segment is unused)
        float sc = run;
        float y = dpp_mov<0x111>(sc);  // row_shr:1
        if (part >= 1) sc += y;
        y = dpp_mov<0x112>(sc);        // row_shr:2
        if (part >= 2) sc += y;
        y = dpp_mov<0x114>(sc);        // row_shr:4
        if (part >= 4) sc += y;
        const float scx = dpp_mov<0x111>(sc);
        const float off = part > 0 ? scx : 0.f;  // the earlier parts of the row (one-lane shift, no subtraction)
        *reinterpret_cast<float4 *>(row) = make_float4(ex[0] + off, ex[1] + off, ex[2] + off, ex[3] + off);
        *reinterpret_cast<float4 *>(row + 4) = make_float4(ex[4] + off, ex[5] + off, ex[6] + off, ex[7] + off);
    }
    __syncthreads();
    {
        const int u = tid >> 3, k = tid & 7;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 8 * k + i;
            acc += r >= u ? sE[r * LDC + u] : 0.f;
        }
        acc += dpp_mov<DPP_QUAD_1032>(acc);
        acc += dpp_mov<DPP_QUAD_2301>(acc);
        acc += dpp_mov<DPP_ROW_HALF_MIRROR>(acc);  // the other quad of the 8-lane group
        if (k == 0 && u < n) {
            const size_t gi = g0 + (size_t)u * a.Hv;
            float dgv = acc + sScan[0][u] + sScan[1][u];
            if (a.gate == GATE_DECAY) dgv = dg_per_decay(dgv, a.g[gi]);
            a.dg[gi] = dgv;
        }
    }
}

// dG bookkeeping.  Every term of the log-decay gradient depends on a difference G_r - G_s' of cumulative log
// decays (s' = -1 stands for the chunk start), so it is a "pair" term E[r][s'] that adds +E to dG_r and -E to
// dG_s'.  The gradient of the per-token log decay g_u is then the sum of the pair terms whose span straddles
// u:  dg_u = sum_{r >= u} sum_{s' < u} E[r][s'].  Summing only straddling terms (each carrying the factor
// exp(g_u)) keeps dg accurate for tiny decays, where a reverse cumulative sum of dG would cancel.

// One value head hv = hk * rep + rr of key head hk.  dq | dk of the key head are summed in order (rr = 0, 1, ...)
// in the part rows of its first value head hk * rep, each thread reading back only the elements it wrote itself,
// and the last value head writes dq and dk in the gradient dtype.  T and dDelta enter only through TdD = T^T dDelta
// (saved by ck_bwd_seq_kernel): dv = diag(beta) TdD, dK -= diag(beta gamma) Y2 (Y2 = TdD h^T), dA = -TdD Delta^T
// below the diagonal, dbeta += rowsum(V * TdD) - gamma s4 and dG -= beta gamma s4 (s4 = rowsum(K * Y2)).
template <bool AF32>
__device__ __forceinline__ void bwd_local_f32_head(const Args &a, int c, int hk, int b, int rr, int rep) {
    DTYPES_OF(a);
    __shared__ __align__(16) float R1[D * LD];       // h, then dh' ([j][i]); then K at R1, Q at R1 + C*LD
    __shared__ __align__(16) float R2[C * LD];       // dY, then the pair matrix E
    __shared__ __align__(16) float RX[2 * C * LDC];  // TdD, then Delta ([C][LD] fits); R4 = RX + C*LDC: dPG, M
    __shared__ double sG[C];
    __shared__ float sGam[C], sRc[C], sB[C], sVT[C], sScan[2][C];
    __shared__ float sRow[3][2][C];                  // per column half: chunk-start pair terms, t2 terms, dbeta
    __shared__ float sLast[8];

    const bool first = rr == 0, last = rr == rep - 1;
    const int hv = hk * rep + rr;
    // an opaque thread index per value head: the lane-dependent addresses are formed inside the head instead of
    // being hoisted out of the caller's loop and held in registers across the whole head
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int r0 = 16 * (w & 3), ch = w >> 2;  // this wave's rows r0..r0+15 and column half
    const int T = a.T, t0 = c * C, n = min(C, T - t0);
    const size_t ci = chunk_index(a, b, hv, c);
    float *const sKm = R1;
    float *const sQm = R1 + C * LD;
    float *const R4 = RX + C * LDC;
    static_assert(C * LD <= 2 * C * LDC, "a [C][D] tile fits RX");
    const float *Hc = a.w.H + ci * D * D;
    const float *dHc = a.w.dH + ci * D * D;
    const float *Dc = a.w.Dl + ci * C * D;
    const float *TDc = a.w.dDl + ci * C * D;
    const size_t qk0 = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * a.Ts + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;
    const size_t park_row = (size_t)a.Hv * 2 * D;

    // ---- phase 0: gates, dY, h; TdD with dv = diag(beta) TdD and rowsum(V * TdD) from its loads
    if (tid < C) {
        sG[tid] = a.w.G[ci * C + tid];
        const float bt = a.beta[((size_t)b * a.Ts + t0 + min(tid, n - 1)) * a.Hv + hv];
        sB[tid] = tid < n ? bt : 0.f;
    }
    load_tile<D, D, NTB>(R1, LD, Hc, D, D, DT_F32, nullptr, tid);
    load_tile<C, D, NTB>(R2, LD, elem_ptr(a.dy, v0, k_dy_dt), v_row, n, k_dy_dt, nullptr, tid);
    {
        constexpr int PER = C * D / 4 / NTB;  // float4 pieces per thread; 32 consecutive threads hold one row
        static_assert(PER * NTB * 4 == C * D && (D / 4) == 32, "even split, half a wave per row");
        float4 td[PER];
        float vv[PER][4], bt[PER];
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int v = tid + p * NTB, r = v / (D / 4), c4 = (v - r * (D / 4)) * 4;
            td[p] = *reinterpret_cast<const float4 *>(TDc + r * D + c4);
            // rows past n read row n - 1 and are zeroed after: no load sits under a branch
            const int rc = min(r, n - 1);
            const float b4 = a.beta[((size_t)b * a.Ts + t0 + rc) * a.Hv + hv];
            bt[p] = r < n ? b4 : 0.f;
            if constexpr (AF32) {
                const float4 x = *reinterpret_cast<const float4 *>(static_cast<const float *>(a.v) + v0 +
                                                                   (size_t)rc * v_row + c4);
                vv[p][0] = x.x; vv[p][1] = x.y; vv[p][2] = x.z; vv[p][3] = x.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) vv[p][q] = load_as_f32(a.v, v0 + (size_t)rc * v_row + c4 + q, k_in_dt);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) vv[p][q] = r < n ? vv[p][q] : 0.f;
        }
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int v = tid + p * NTB, r = v / (D / 4), c4 = (v - r * (D / 4)) * 4;
            *reinterpret_cast<float4 *>(RX + r * LD + c4) = td[p];
            float vt = vv[p][0] * td[p].x + vv[p][1] * td[p].y + vv[p][2] * td[p].z + vv[p][3] * td[p].w;
            vt = row16_allreduce(vt);
            vt += lane_xor16(vt);
            if ((tid & 31) == 0) sVT[r] = vt;
            if (r < n) {
                const float4 dv = make_float4(bt[p] * td[p].x, bt[p] * td[p].y, bt[p] * td[p].z, bt[p] * td[p].w);
                const size_t o = v0 + (size_t)r * v_row + c4;
                if (k_grad_dt == DT_F32) {
                    *reinterpret_cast<float4 *>(static_cast<float *>(a.dv) + o) = dv;
                } else {
                    store_from_f32(a.dv, o, dv.x, k_grad_dt);
                    store_from_f32(a.dv, o + 1, dv.y, k_grad_dt);
                    store_from_f32(a.dv, o + 2, dv.z, k_grad_dt);
                    store_from_f32(a.dv, o + 3, dv.w, k_grad_dt);
                }
            }
        }
    }
    __syncthreads();
    if (tid < C) {
        sGam[tid] = expf((float)sG[tid]);
        sRc[tid] = expf((float)(sG[C - 1] - sG[tid]));
    }
    float lastp = 0.f;  // pair (C-1, chunk start): gamma_C <dh', h>
    {
        constexpr int PER = D * D / 4 / NTB;
        float4 dv4[PER];
#pragma unroll
        for (int p = 0; p < PER; ++p) dv4[p] = reinterpret_cast<const float4 *>(dHc)[tid + p * NTB];
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int v = tid + p * NTB, i = v / (D / 4), j = (v - i * (D / 4)) * 4;
            const float *hh = R1 + i * LD + j;
            lastp += dv4[p].x * hh[0] + dv4[p].y * hh[1] + dv4[p].z * hh[2] + dv4[p].w * hh[3];
        }
    }
    float bnd[4] = {0.f, 0.f, 0.f, 0.f};   // pair terms (r, chunk start) of rows r0+4lg+e, this lane's columns
    float rowB[4] = {0.f, 0.f, 0.f, 0.f};  // dbeta partials
    float tl[4] = {0.f, 0.f, 0.f, 0.f};    // pair terms (C-1, r)

    // ---- phase 1: dQ = diag(gamma) dY h^T ; Y2 = TdD h^T.  This lane's A values of TdD (row r0 + li, columns
    // 4 k + lg) stay in registers for dA = TdD Delta^T in phase 2.
    f4 dQ[4], dK[4], Y2[4];
    float tdA[D / 4];
    {
#pragma unroll
        for (int t = 0; t < 4; ++t) dQ[t] = Y2[t] = zero4();
        const float *ay = R2 + (r0 + li) * LD + lg, *at = RX + (r0 + li) * LD + lg;
        const float *bh = R1 + (64 * ch + li) * LD + lg;
#pragma unroll 8
        for (int k = 0; k < D / 4; ++k) {
            const float yv = ay[4 * k], tv = at[4 * k];
            tdA[k] = tv;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float bv = bh[16 * t * LD + 4 * k];
                dQ[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(yv, bv, dQ[t], 0, 0, 0);
                Y2[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(tv, bv, Y2[t], 0, 0, 0);
            }
        }
    }
    __syncthreads();  // sGam / sRc ready; phase 1's tiles read
    // the waves' parts of <dh', h> go to LDS now
    lastp = wave_sum(lastp * sGam[C - 1]);
    if (l == 0) sLast[w] = lastp;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) dQ[t][e] *= sGam[r0 + 4 * lg + e];
    // ---- phase 2: dK = diag(gamma_C/gamma) Delta dh'^T ; dP = lower(dY Delta^T) ; dA = -TdD Delta^T
    load_tile<D, D, NTB>(R1, LD, dHc, D, D, DT_F32, nullptr, tid);
    load_tile<C, D, NTB>(RX, LD, Dc, D, C, DT_F32, nullptr, tid);  // Delta in place of TdD (phase 1 is done)
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; ++t) dK[t] = zero4();
    mma_strip<D, 4>(dK, RX + r0 * LD, LD, 1, R1 + 64 * ch * LD, 1, LD, 16 * LD, l);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) dK[t][e] *= sRc[r0 + 4 * lg + e];
    f4 dPG[2], Ep[2], dA[2];
    {
        // this lane's P values, loaded before the products and with no branch (the C x C tile holds every (r, s))
        float pw[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                pw[t][e] = a.w.P[ci * C * C + (r0 + 4 * lg + e) * C + 32 * ch + 16 * t + li];
        f4 dp[2] = {zero4(), zero4()};
        dA[0] = dA[1] = zero4();
        mma_strip<D, 2>(dp, R2 + r0 * LD, LD, 1, RX + 32 * ch * LD, 1, LD, 16 * LD, l);
        const float *bd = RX + (32 * ch + li) * LD + lg;
#pragma unroll 8
        for (int k = 0; k < D / 4; ++k)
#pragma unroll
            for (int t = 0; t < 2; ++t)
                dA[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(tdA[k], bd[16 * t * LD + 4 * k], dA[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = r0 + 4 * lg + e, s2 = 32 * ch + 16 * t + li;
                const float pv = s2 <= r ? dp[t][e] : 0.f;
                Ep[t][e] = s2 < r ? pv * pw[t][e] : 0.f;
                dPG[t][e] = s2 <= r ? pv * expf((float)(sG[r] - sG[s2])) : 0.f;
            }
    }
    __syncthreads();
    // ---- phase 3: dQ += dPG K ; dK += dPG^T Q ; K K^T
    load_tile<C, D, NTB>(sKm, LD, elem_ptr(a.k, qk0, k_in_dt), qk_row, n, k_in_dt, nullptr, tid);
    load_tile<C, D, NTB>(sQm, LD, elem_ptr(a.q, qk0, k_in_dt), qk_row, n, k_in_dt, nullptr, tid);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) R4[(r0 + 4 * lg + e) * LDC + 32 * ch + 16 * t + li] = dPG[t][e];
    __syncthreads();
    // the boundary terms q . dQ and k . dK (before the products), and Z's terms through Y2: s4 = k . Y2
    // (dbeta -= gamma s4, dG -= beta gamma s4), dK -= beta gamma Y2
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = r0 + 4 * lg + e, j = 64 * ch + 16 * t + li;
            const float kv = sKm[r * LD + j], bg = sB[r] * sGam[r];
            bnd[e] += sQm[r * LD + j] * dQ[t][e];
            tl[e] += kv * dK[t][e];
            const float s4 = kv * Y2[t][e];
            rowB[e] -= sGam[r] * s4;
            bnd[e] -= bg * s4;
            dK[t][e] -= bg * Y2[t][e];
        }
    mma_strip<C, 4>(dQ, R4 + r0 * LDC, LDC, 1, sKm + 64 * ch, LD, 1, 16, l);
    mma_strip<C, 4>(dK, R4 + r0, 1, LDC, sQm + 64 * ch, LD, 1, 16, l);
    f4 Mt[2];
    {
        f4 kk[2] = {zero4(), zero4()};
        mma_strip<D, 2>(kk, sKm + r0 * LD, LD, 1, sKm + 32 * ch * LD, 1, LD, 16 * LD, l);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = r0 + 4 * lg + e, s2 = 32 * ch + 16 * t + li;
                const float gam = s2 < r ? expf((float)(sG[r] - sG[s2])) : 0.f;
                const float dav = s2 < r ? -dA[t][e] : 0.f;
                const float kg = kk[t][e] * gam;
                rowB[e] += dav * kg;
                Ep[t][e] += dav * sB[r] * kg;
                Mt[t][e] = sB[r] * dav * gam;
            }
    }
    __syncthreads();
    // ---- phase 4: dK += (M + M^T) K
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) R4[(r0 + 4 * lg + e) * LDC + 32 * ch + 16 * t + li] = Mt[t][e];
    __syncthreads();
    mma_strip<C, 4>(dK, R4 + r0 * LDC, LDC, 1, sKm + 64 * ch, LD, 1, 16, l);
    mma_strip<C, 4>(dK, R4 + r0, 1, LDC, sKm + 64 * ch, LD, 1, 16, l);
    // ---- phase 6: straddle sums for dg, dbeta, outputs.  R2 (dY) is free: E goes there.
    float *const sE = R2;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) sE[(r0 + 4 * lg + e) * LDC + 32 * ch + 16 * t + li] = Ep[t][e];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float bsum = row16_allreduce(bnd[e]);
        const float t2 = row16_allreduce(tl[e]);
        const float rbv = row16_allreduce(rowB[e]);
        const int r = r0 + 4 * lg + e;
        if (li == 0) {
            sRow[0][ch][r] = bsum;
            sRow[1][ch][r] = t2;
            sRow[2][ch][r] = ch == 0 ? rbv + sVT[r] : rbv;
        }
    }
    __syncthreads();
    // dq and dk leave through a wave-private staging block in R1 (free after the barrier above: the wave's 16 x 64
    // fp32 part, row stride LQ), one matrix after the other: each lane moves four 16-byte row pieces per matrix
    // (piece p: row (l + 64p) / 16, columns 4 ((l + 64p) % 16) .. +3) instead of 16 scattered 4-byte elements.
    // The running dq | dk sum of the previous value heads at those pieces is in flight during the sums.
    constexpr int LQ = 64 + 4;
    static_assert(8 * 16 * LQ <= D * LD, "staging fits R1");
    float *const stg = R1 + w * 16 * LQ;
    float *const sum_row = a.w.part + ((size_t)b * T + t0) * a.Hv * 2 * D + (size_t)hk * rep * 2 * D;
    float4 prq[4], prk[4];
    if (!first) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int i = l + 64 * p, r = r0 + (i >> 4), c4 = 64 * ch + 4 * (i & 15);
            const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            const int rc = min(r, n - 1);  // rows past n read row n - 1, unused: no load under a branch
            const float4 xq = *reinterpret_cast<const float4 *>(sum_row + (size_t)rc * park_row + c4);
            const float4 xk = *reinterpret_cast<const float4 *>(sum_row + (size_t)rc * park_row + D + c4);
            prq[p] = r < n ? xq : z;
            prk[p] = r < n ? xk : z;
        }
    }
    chunk_dg_dbeta<NTB>(sE, sRow, sLast, 1.f, sScan, a, b, hv, t0, n, tid);
    const size_t qk_out = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D;
    auto out = [&](const f4 (&X)[4], const float4 (&prev)[4], int half, void *dst) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) stg[(4 * lg + e) * LQ + 16 * t + li] = X[t][e];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int i = l + 64 * p, rr2 = i >> 4, r = r0 + rr2, c4 = 64 * ch + 4 * (i & 15);
            float4 v = *reinterpret_cast<const float4 *>(stg + rr2 * LQ + 4 * (i & 15));
            if (r >= n) continue;
            if (!first) v = make_float4(prev[p].x + v.x, prev[p].y + v.y, prev[p].z + v.z, prev[p].w + v.w);
            const size_t o = qk_out + (size_t)r * a.Hk * D + c4;
            if (!last) {
                *reinterpret_cast<float4 *>(sum_row + (size_t)r * park_row + half * D + c4) = v;
            } else if (k_grad_dt == DT_F32) {
                *reinterpret_cast<float4 *>(static_cast<float *>(dst) + o) = v;
            } else {
                store_from_f32(dst, o, v.x, k_grad_dt);
                store_from_f32(dst, o + 1, v.y, k_grad_dt);
                store_from_f32(dst, o + 2, v.z, k_grad_dt);
                store_from_f32(dst, o + 3, v.w, k_grad_dt);
            }
        }
    };
    out(dQ, prq, 0, a.dq);
    out(dK, prk, 1, a.dk);
    __syncthreads();  // the pair matrix read: the next value head's tiles reuse its space
}

// One workgroup of 8 waves per (chunk, key head), walking the key head's value heads in order.
template <bool AF32>
__global__ __launch_bounds__(NTB) void ck_bwd_local_kernel(Args a) {
    typedef const __attribute__((address_space(4))) Args *KArgs;  // the kernel arguments (constant memory)
    const int rep = a.Hv / a.Hk;
    for (int rr = 0; rr < rep; ++rr) {
        // the arguments are read anew for each value head instead of being held in scalar registers across it
        KArgs ap = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
        asm volatile("" : "+s"(ap));
        bwd_local_f32_head<AF32>(*(const Args *)ap, blockIdx.x, blockIdx.y, blockIdx.z, rr, rep);
    }
}


// ---------------------------------------------------------------------------------------------- ck_bwd_local (bf16)
//
// One workgroup of 8 waves per (chunk, key head) takes the key head's value heads in turn; for each, wave w owns
// the 16-row strip r0 = 16 (w % 4) and column half w / 4 of every [64][*] product.  T and dDelta enter only through
// TdD = T^T dDelta, which ck_bwd_seq_bf16 saves: with Delta = T Z, Z = diag(beta) V - diag(beta gamma) K h,
//   dv = diag(beta) TdD,   dK -= diag(beta gamma) Y2 (Y2 = TdD h^T),   dA = -strict_lower(TdD Delta^T),
//   dbeta += rowsum(V * TdD) - gamma s4,   dG -= beta gamma s4   (s4 = rowsum(K * Y2)).
// Phases and their tiles (byte offsets into one LDS arena; lifetimes checked against the barriers between phases):
//   S1  dQ = gamma dY h^T, Y2 = TdD h^T, dK = rc Delta dh'^T, dp = dY Delta^T, dA = TdD Delta^T in one pass over
//       the value index (Delta split; TdD as bf16, dv and rowsum(V * TdD) from its fp32 loads)
//                                                                  TdD, h, dh', Delta hi / lo, dY
//   S3  dQ += dPG K, dK += dPG^T Q (dPG split), K K^T               dPG, dPG^T, Q^T, K^T, K
//   S6  dK += M K + M^T K, M = diag(beta) dA * Gam                   M, M^T, K^T
// then the straddle sums for dg and the outputs, as in ck_bwd_local_kernel.
constexpr int SZ_A = C * LA * 2;       // [64][136]  17408 B
constexpr int SZ_B = D * LA * 2;       // [128][136] 34816 B
constexpr int SZ_C = D * LB * 2;       // [128][72]  18432 B
constexpr int SZ_D = C * LB * 2;       // [64][72]    9216 B
constexpr int LQ = 64 + 4;             // row stride of a wave's fp32 dq staging block
// S1: TdD, dh', h, Delta hi / lo, dY
constexpr int O_TD = 0;
constexpr int O_DHH = O_TD + SZ_A, O_H = O_DHH + SZ_B, O_DLH = O_H + SZ_B, O_DLL = O_DLH + SZ_A;
constexpr int O_DY = O_DLL + SZ_A;
// S3: dPG, dPG^T (hi / lo), Q^T, K^T, K, then the waves' dq staging blocks
constexpr int O_PNH = 0, O_PNL = O_PNH + SZ_D, O_PTH = O_PNL + SZ_D, O_PTL = O_PTH + SZ_D;
constexpr int O_QT = O_PTL + SZ_D, O_KT = O_QT + SZ_C, O_K = O_KT + SZ_C, O_STQ = O_K + SZ_A;
// S6: M and M^T (bf16) over the dead dPG tiles; then the pair matrix E over the dq staging
constexpr int O_MM = 0, O_MT = O_MM + SZ_D, O_SM = O_STQ;
constexpr int ARENA = O_DY + SZ_A;
static_assert(O_STQ + 8 * 16 * LQ * 4 <= ARENA, "dq staging fits");
static_assert(O_SM + C * LDC * 4 <= ARENA && O_MT + SZ_D <= O_QT, "S6 tiles fit, clear of K^T");
static_assert(C * (D + 4) * 4 <= O_KT, "dk staging below K^T and the pair matrix");

constexpr int NQR = 4;  // dq row pieces per thread whose running sum stays in registers (of four: all of them)

// One value head hv = hk * rep + rr of key head hk.  dq | dk of the key head: the value heads' fp32 parts are summed
// in order (rr = 0, 1, ...) at the 16-byte row pieces each thread writes out: dk (ck) and the first NQR dq pieces
// (cq) in registers, any other dq pieces in the part rows of the key head (each thread reading back only the
// elements it wrote itself); the last value head writes dq and dk in the gradient dtype.
template <bool DYF32>
__device__ __forceinline__ void bwd_local_bf16_head(const Args &a, int c, int hk, int b, int rr, int rep,
                                                    float4 (&ck)[4], float4 (&cq)[NQR]) {
    __shared__ __align__(16) unsigned char arena[ARENA];
    __shared__ double sG[C];
    __shared__ float sGam[C], sRc[C], sB[C], sVT[C], sScan[2][C];
    __shared__ float sRow[3][2][C];
    __shared__ float sLast[8];
    auto T16 = [&](int off) { return reinterpret_cast<bfr *>(arena + off); };

    const bool first = rr == 0, last = rr == rep - 1;
    const int hv = hk * rep + rr;
    const int T = a.T, t0 = c * C, n = min(C, T - t0);
    float *const part_row = a.w.part + (((size_t)b * T + t0) * a.Hk + hk) * 2 * D;
    const size_t part_rs = (size_t)a.Hk * 2 * D;
    const size_t qk_out = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D;
    // an opaque lane index per value head: the lane-dependent addresses are formed inside the head instead of
    // being hoisted out of the caller's loop and held in registers across the whole head
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int r0 = 16 * (w & 3), ch = w >> 2;
    const size_t ci = chunk_index(a, b, hv, c);
    const bfr *Hc = reinterpret_cast<const bfr *>(a.w.H) + ci * D * D;    // h = S^T, [j][i], bf16
    const bfr *dHc = reinterpret_cast<const bfr *>(a.w.dH) + ci * D * D;  // dh', [j][i], bf16
    const float *Dc = a.w.Dl + ci * C * D;                                // Delta [r][i]
    const float *TDc = a.w.dDl + ci * C * D;                              // TdD [r][i]
    const size_t qk0 = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * a.Ts + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;
    const bfr *qsrc = static_cast<const bfr *>(a.q) + qk0, *ksrc = static_cast<const bfr *>(a.k) + qk0;
    const bfr *vsrc = static_cast<const bfr *>(a.v) + v0;

    // ---- S1 staging: gates; h, dh', Delta, TdD, dY, V.  Every global load of the phase is issued before the
    // first LDS store, the gates' too, and the dtype of dY is a template parameter: a gate stored to LDS before
    // the tile loads, or a branch on the dtype among them, made the compiler wait for the loads in flight and split
    // the phase's loads into serial batches.  dv = diag(beta) TdD leaves from the fp32 TdD loads, and
    // rowsum(V * TdD) goes to sVT.
    double gch = 0.0;
    float bch = 0.f;
    if (tid < C) {
        gch = a.w.G[ci * C + tid];
        bch = tid < n ? a.beta[((size_t)b * a.Ts + t0 + tid) * a.Hv + hv] : 0.f;
    }
    float lastp = 0.f;  // <dh', h>, the pair (C-1, chunk start)
    {
        constexpr int SPER = D * (D / 8) / NTB, NPER = C * (D / 8) / NTB;  // 8-element pieces per thread
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
            vr[p] = r < n ? *reinterpret_cast<const uint4 *>(vsrc + (size_t)r * v_row + c8) : make_uint4(0u, 0u, 0u, 0u);
            bt[p] = r < n ? a.beta[((size_t)b * a.Ts + t0 + r) * a.Hv + hv] : 0.f;
            if constexpr (DYF32) {
                const float *ys = static_cast<const float *>(a.dy) + v0 + (size_t)r * v_row + c8;
                yr[2 * p] = r < n ? *reinterpret_cast<const uint4 *>(ys) : make_uint4(0u, 0u, 0u, 0u);
                yr[2 * p + 1] = r < n ? *reinterpret_cast<const uint4 *>(ys + 4) : make_uint4(0u, 0u, 0u, 0u);
            } else {
                yr[p] = r < n ? *reinterpret_cast<const uint4 *>(static_cast<const bfr *>(a.dy) + v0 + (size_t)r * v_row + c8)
                              : make_uint4(0u, 0u, 0u, 0u);
            }
        }
        if (tid < C) {
            sG[tid] = gch;
            sB[tid] = bch;
        }
        bfr *const th = T16(O_H), *const tdh = T16(O_DHH);
#pragma unroll
        for (int p = 0; p < SPER; ++p) {
            const int pc = tid + p * NTB, r = pc / (D / 8), c8 = (pc - r * (D / 8)) * 8;
            *reinterpret_cast<uint4 *>(th + r * LA + c8) = hr[p];
            *reinterpret_cast<uint4 *>(tdh + r * LA + c8) = dhr[p];
            const uint32_t hw[4] = {hr[p].x, hr[p].y, hr[p].z, hr[p].w}, dw[4] = {dhr[p].x, dhr[p].y, dhr[p].z, dhr[p].w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                lastp += bf2f(hw[q] & 0xffffu) * bf2f(dw[q] & 0xffffu) + bf2f(hw[q] >> 16) * bf2f(dw[q] >> 16);
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
            *reinterpret_cast<uint4 *>(T16(O_DLH) + r * LA + c8) = h;
            *reinterpret_cast<uint4 *>(T16(O_DLL) + r * LA + c8) = lo;
            const uint4 t0v = td[2 * p], t1v = td[2 * p + 1];
            const float tv[8] = {f(t0v.x), f(t0v.y), f(t0v.z), f(t0v.w), f(t1v.x), f(t1v.y), f(t1v.z), f(t1v.w)};
            *reinterpret_cast<uint4 *>(T16(O_TD) + r * LA + c8) =
                make_uint4(pk(tv[0], tv[1]), pk(tv[2], tv[3]), pk(tv[4], tv[5]), pk(tv[6], tv[7]));
            uint4 yv;
            if constexpr (DYF32) {
                const uint4 y0 = yr[2 * p], y1 = yr[2 * p + 1];
                yv = make_uint4(pk(f(y0.x), f(y0.y)), pk(f(y0.z), f(y0.w)), pk(f(y1.x), f(y1.y)), pk(f(y1.z), f(y1.w)));
            } else {
                yv = yr[p];
            }
            *reinterpret_cast<uint4 *>(T16(O_DY) + r * LA + c8) = yv;
            // rowsum(V * TdD): the 16 lanes of a DPP row hold one token's row
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
    // the waves' parts of <dh', h> go to LDS now (the raw h / dh' loads are not kept live until the straddle sums)
    lastp = wave_sum(lastp);
    if (l == 0) sLast[w] = lastp;
    __syncthreads();
    if (tid < C) {
        sGam[tid] = expf((float)sG[tid]);
        sRc[tid] = expf((float)(sG[C - 1] - sG[tid]));
    }
    // S3's Q^T (threads 0-255) and K, K^T (threads 256-511) blocks, in flight during the S1 products: one 8 x 4
    // block per thread
    constexpr int NBQ = (C / 8) * (D / 4);
    static_assert(2 * NBQ == NTB, "one block per thread");
    const bool isk = tid >= NBQ;
    Blk84 bk;
    bk.load(isk ? ksrc : qsrc, qk_row, isk ? tid - NBQ : tid, D, n);
    float bnd[4] = {0.f, 0.f, 0.f, 0.f}, rowB[4] = {0.f, 0.f, 0.f, 0.f}, tl[4] = {0.f, 0.f, 0.f, 0.f};
    f4 dQ[4], dK[4], Y2[4], dPG[2], Ep[2], dA[2];
#pragma unroll
    for (int t = 0; t < 4; ++t) dQ[t] = dK[t] = Y2[t] = zero4();
    {
        f4 dp[2] = {zero4(), zero4()};
#pragma unroll
        for (int t = 0; t < 2; ++t) dA[t] = zero4();
        // one pass over the value index: each fragment read from LDS once per k-step (dQ and Y2 share the h
        // fragments, dp and dA the Delta fragments)
        const bfr *const tY = T16(O_DY), *const tT = T16(O_TD), *const tH = T16(O_H), *const tDH = T16(O_DHH);
        const bfr *const tLh = T16(O_DLH), *const tLl = T16(O_DLL);
#pragma unroll 2
        for (int k0 = 0; k0 < D; k0 += 32) {
            const bf8 ay = frag(tY, LA, r0, k0, l), at = frag(tT, LA, r0, k0, l);
            const bf8 ah = frag(tLh, LA, r0, k0, l), al = frag(tLl, LA, r0, k0, l);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf8 hb = frag(tH, LA, 64 * ch + 16 * t, k0, l);
                dQ[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ay, hb, dQ[t], 0, 0, 0);
                Y2[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at, hb, Y2[t], 0, 0, 0);
                const bf8 db = frag(tDH, LA, 64 * ch + 16 * t, k0, l);
                dK[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, db, dK[t], 0, 0, 0);
                dK[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, db, dK[t], 0, 0, 0);
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const bf8 xh = frag(tLh, LA, 32 * ch + 16 * t, k0, l), xl = frag(tLl, LA, 32 * ch + 16 * t, k0, l);
                dp[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ay, xh, dp[t], 0, 0, 0);
                dp[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ay, xl, dp[t], 0, 0, 0);
                dA[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at, xh, dA[t], 0, 0, 0);
                dA[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(at, xl, dA[t], 0, 0, 0);
            }
        }
        __syncthreads();  // sGam / sRc ready; the S1 tiles read
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dQ[t][e] *= sGam[r0 + 4 * lg + e];
                dK[t][e] *= sRc[r0 + 4 * lg + e];
            }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = r0 + 4 * lg + e, s2 = 32 * ch + 16 * t + li;
                const float pv = s2 <= r ? dp[t][e] : 0.f;
                Ep[t][e] = s2 < r ? pv : 0.f;  // times P below
                dPG[t][e] = s2 <= r ? pv * __builtin_amdgcn_exp2f((float)(sG[r] - sG[s2]) * 1.4426950408889634f) : 0.f;
            }
    }
    // ---- S3: dQ += dPG K, dK += dPG^T Q, K K^T
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        acc_N<true>(dPG[t], T16(O_PNH), T16(O_PNL), LB, r0, 32 * ch + 16 * t, l);
        acc_T<true>(dPG[t], T16(O_PTH), T16(O_PTL), LB, r0, 32 * ch + 16 * t, l);
    }
    if (isk) {
        bk.store_N(T16(O_K), LA);
        bk.store_T(T16(O_KT), LB);
    } else {
        bk.store_T(T16(O_QT), LB);
    }
    // dQ leaves through a wave-private staging block (the wave's 16 x 64 fp32 part of dQ, row stride LQ): each lane
    // then moves four 16-byte row pieces (piece p: row (l + 64p) / 16, columns 4 ((l + 64p) % 16) .. +3) instead of
    // 16 scattered 4-byte elements.  The running dq sum of the previous value heads at those pieces, and P at this
    // lane's pair positions, are in flight during the S3 products.
    float *const stq = reinterpret_cast<float *>(arena + O_STQ) + w * 16 * LQ;
    float4 prevq[4];
    if (!first) {
#pragma unroll
        for (int p = NQR; p < 4; ++p) {
            const int i = l + 64 * p, r = r0 + (i >> 4), c4 = 64 * ch + 4 * (i & 15);
            prevq[p] = r < n ? *reinterpret_cast<const float4 *>(part_row + (size_t)r * part_rs + c4)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    // P at (r = r0 + 4 lg + e, s = 32 ch + 16 t + li), read from the P^T tile (fragment order), where the four rows
    // of one column are 8 contiguous bytes per plane
    uint2 pP[2][2];  // [t][hi, lo]
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const size_t pi = ci * 2 * C * C + frag_off<C>(32 * ch + 16 * t + li, r0 + 4 * lg);
        pP[t][0] = *reinterpret_cast<const uint2 *>(a.w.PTb + pi);
        pP[t][1] = *reinterpret_cast<const uint2 *>(a.w.PTb + pi + C * C);
    }
    __syncthreads();
    {
        // the boundary terms q . dQ and k . dK (before the S3 products), and Z's terms through Y2 = TdD h^T:
        // s4 = k . Y2 (dbeta -= gamma s4, dG -= beta gamma s4), dK -= beta gamma Y2
        const bfr *Qt = T16(O_QT), *Kt = T16(O_KT);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = r0 + 4 * lg + e, j = 64 * ch + 16 * t + li;
                const float kv = bf2f(Kt[j * LB + r]), bg = sB[r] * sGam[r];
                bnd[e] += bf2f(Qt[j * LB + r]) * dQ[t][e];
                tl[e] += kv * dK[t][e];
                const float s4 = kv * Y2[t][e];
                rowB[e] -= sGam[r] * s4;
                bnd[e] -= bg * s4;
                dK[t][e] -= bg * Y2[t][e];
            }
    }
    mmab<C, 4, true>(dQ, T16(O_PNH), T16(O_PNL), LB, r0, T16(O_KT), nullptr, LB, 64 * ch, l);
    mmab<C, 4, true>(dK, T16(O_PTH), T16(O_PTL), LB, r0, T16(O_QT), nullptr, LB, 64 * ch, l);
    // dQ is complete: it goes out now (to the running sum, or as dq from the last value head) instead of staying
    // live
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) stq[(4 * lg + e) * LQ + 16 * t + li] = dQ[t][e];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const int i = l + 64 * p, rr2 = i >> 4, r = r0 + rr2, c4 = 64 * ch + 4 * (i & 15);
        float4 v = *reinterpret_cast<const float4 *>(stq + rr2 * LQ + 4 * (i & 15));
        if (r >= n) continue;
        if (!first) {
            const float4 s = p < NQR ? cq[p < NQR ? p : 0] : prevq[p];
            v = make_float4(s.x + v.x, s.y + v.y, s.z + v.z, s.w + v.w);
        }
        const size_t o = qk_out + (size_t)r * a.Hk * D + c4;
        if (!last) {
            if (p < NQR) cq[p < NQR ? p : 0] = v;
            else *reinterpret_cast<float4 *>(part_row + (size_t)r * part_rs + c4) = v;
        } else if (a.grad_dt == DT_BF16) {
            *reinterpret_cast<uint2 *>(static_cast<bfr *>(a.dq) + o) = make_uint2(pk(v.x, v.y), pk(v.z, v.w));
        } else if (a.grad_dt == DT_F32) {
            *reinterpret_cast<float4 *>(static_cast<float *>(a.dq) + o) = v;
        } else {
            store_from_f32(a.dq, o, v.x, a.grad_dt);
            store_from_f32(a.dq, o + 1, v.y, a.grad_dt);
            store_from_f32(a.dq, o + 2, v.z, a.grad_dt);
            store_from_f32(a.dq, o + 3, v.w, a.grad_dt);
        }
    }
    // A's terms: dA = -TdD Delta^T strictly below the diagonal; dbeta += dA . (K K^T * Gam), the pair terms
    // E += P * dP + dA * A, M = diag(beta) dA * Gam (K K^T after dQ has left: fewer accumulators live)
    f4 kk[2] = {zero4(), zero4()};
    mmab<D, 2>(kk, T16(O_K), nullptr, LA, r0, T16(O_K), nullptr, LA, 32 * ch, l);
    f4 Mt[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = r0 + 4 * lg + e, s2 = 32 * ch + 16 * t + li;
            const float gam = s2 < r ? __builtin_amdgcn_exp2f((float)(sG[r] - sG[s2]) * 1.4426950408889634f) : 0.f;
            const float dav = s2 < r ? -dA[t][e] : 0.f;
            const float kg = kk[t][e] * gam;
            rowB[e] += dav * kg;
            const auto half = [e](uint2 v) { const uint32_t x = e < 2 ? v.x : v.y; return bf2f(e & 1 ? x >> 16 : x & 0xffffu); };
            Ep[t][e] = Ep[t][e] * (half(pP[t][0]) + half(pP[t][1])) + dav * sB[r] * kg;
            Mt[t][e] = sB[r] * dav * gam;
        }
    __syncthreads();  // dPG, Q^T and the dq staging read (K^T stays)
    // ---- S6: dK += (M + M^T) K.  M is strictly lower triangular, so M and M^T never overlap: the bf16 tiles of M
    // and of M^T, written from the accumulators in both orientations, are exactly the rounded M + M^T, and the two
    // products (the second A operand in mmab's lo slot) replace a pairing pass over an fp32 copy of M
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        acc_N<false>(Mt[t], T16(O_MM), nullptr, LB, r0, 32 * ch + 16 * t, l);
        acc_T<false>(Mt[t], T16(O_MT), nullptr, LB, r0, 32 * ch + 16 * t, l);
    }
    __syncthreads();
    mmab<C, 4, true>(dK, T16(O_MM), T16(O_MT), LB, r0, T16(O_KT), nullptr, LB, 64 * ch, l);
    __syncthreads();  // M, M^T and K^T read: the pair matrix E takes the dq staging space, the dk staging the space below
    // dK staged as fp32 rows in the free arena for 16-byte stores
    float *const sp = reinterpret_cast<float *>(arena);
    constexpr int LP = D + 4, PER = C * D / 4 / NTB;
    static_assert(PER * NTB * 4 == C * D, "even split");
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) sp[(r0 + 4 * lg + e) * LP + 64 * ch + 16 * t + li] = dK[t][e];
    // ---- straddle sums for dg, dbeta, outputs
    float *const sE = reinterpret_cast<float *>(arena + O_SM);  // [64][LDC] fp32
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) sE[(r0 + 4 * lg + e) * LDC + 32 * ch + 16 * t + li] = Ep[t][e];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float bsum = row16_allreduce(bnd[e]);
        const float t2 = row16_allreduce(tl[e]);
        const float rbv = row16_allreduce(rowB[e]);
        const int r = r0 + 4 * lg + e;
        if (li == 0) {
            sRow[0][ch][r] = bsum;
            sRow[1][ch][r] = t2;
            sRow[2][ch][r] = ch == 0 ? rbv + sVT[r] : rbv;
        }
    }
    __syncthreads();
    chunk_dg_dbeta<NTB>(sE, sRow, sLast, sGam[C - 1], sScan, a, b, hv, t0, n, tid);
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int i = tid + p * NTB, r = i / (D / 4), c4 = (i - r * (D / 4)) * 4;
        if (r >= n) continue;
        float4 v = *reinterpret_cast<const float4 *>(sp + r * LP + c4);
        if (!first) v = make_float4(ck[p].x + v.x, ck[p].y + v.y, ck[p].z + v.z, ck[p].w + v.w);
        const size_t o = qk_out + (size_t)r * a.Hk * D + c4;
        if (!last) {
            ck[p] = v;
        } else if (a.grad_dt == DT_BF16) {
            *reinterpret_cast<uint2 *>(static_cast<bfr *>(a.dk) + o) = make_uint2(pk(v.x, v.y), pk(v.z, v.w));
        } else if (a.grad_dt == DT_F32) {
            *reinterpret_cast<float4 *>(static_cast<float *>(a.dk) + o) = v;
        } else {
            store_from_f32(a.dk, o, v.x, a.grad_dt);
            store_from_f32(a.dk, o + 1, v.y, a.grad_dt);
            store_from_f32(a.dk, o + 2, v.z, a.grad_dt);
            store_from_f32(a.dk, o + 3, v.w, a.grad_dt);
        }
    }
    __syncthreads();  // the staging tile read: the next value head's tiles reuse the arena
}

// One workgroup of 8 waves per (chunk, key head), walking the key head's value heads in order.
template <bool DYF32>
__global__ __launch_bounds__(NTB) void ck_bwd_local_bf16_kernel(Args a) {
    typedef const __attribute__((address_space(4))) Args *KArgs;  // the kernel arguments (constant memory)
    const int rep = a.Hv / a.Hk;
    float4 ck[4], cq[NQR];  // the running dk and dq sums of the value heads done so far
    static_assert(C * D / 4 / NTB == 4, "four dk row pieces per thread");
    for (int rr = 0; rr < rep; ++rr) {
        // the arguments are read anew for each value head instead of being held in scalar registers across it
        KArgs ap = (KArgs)__builtin_amdgcn_kernarg_segment_ptr();
        asm volatile("" : "+s"(ap));
        bwd_local_bf16_head<DYF32>(*(const Args *)ap, blockIdx.x, blockIdx.y, blockIdx.z, rr, rep, ck, cq);
    }
}

// ---------------------------------------------------------------------------------------------- ck_fwd (bf16)
//
// Sequential over chunks like ck_fwd_kernel, for bf16 inputs.  The A operands of every product (W, Q, P hi / lo,
// (K diag(gamma_C/gamma))^T) are read as MFMA fragments straight from global memory into registers, one chunk
// ahead (ck_prep wrote them as bf16 tiles); LDS only carries what the waves exchange each chunk: h as the
// operand [i][j] (hi / lo) and Delta as [i][r] (hi / lo).  Two barriers per chunk.

template <int DN>
struct FwdFrags {
    bf8 W[4], Q[4], P[4], K[2];  // P[0..1] hi, P[2..3] lo
    float U[DN][4];
    double g;
    float4 gc;  // per-channel gates: G_C of this lane's four state rows
};

// VG: one decay per key channel (gdn_chunk_vg.hip wrote the tiles): Y = (Q * exp(G)) h + P Delta with the Q * exp(G)
// tile as the A operand, and h' = diag(exp(G_C)) h + (K * exp(G_C - G))^T Delta, a decay per state row.
template <int VS, int MODE, bool VG = false>
__global__ __launch_bounds__(NTS) void ck_fwd_bf16_kernel(Args a) {
    constexpr bool kTiles = MODE != FWD_ONLY, kOut = MODE != FWD_RECOMPUTE;
    constexpr int NTN = VS / 16, DN = NTN >= 2 ? NTN / 2 : 1;
    constexpr int LH = D + 8, LDd = C + 8;
    __shared__ __align__(16) bfr sHh[VS * LH];
    __shared__ __align__(16) bfr sHl[VS * LH];
    __shared__ __align__(16) bfr sDh[VS * LDd];
    __shared__ __align__(16) bfr sDl[VS * LDd];
    __shared__ float sGamBuf[2][C];  // by chunk parity: read after the second barrier, rewritten two chunks later

    const SeqBlock sb = seq_block();
    const SeqRange sr = seq_range<MODE>(a, sb.b);
    const int i0 = sb.slice * VS, hv = sb.hv, b = sr.b, cb = sr.cb, ce = sr.ce;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk);
    const size_t head = (size_t)b * a.Hv + hv;
    const int mrow = 16 * (w & 3);
    // with 16-wide slices (NTN == 1) waves 0-3 form Delta and waves 4-7 form y on the same row blocks; wider slices
    // give every wave both
    const bool dwave = NTN >= 2 || w < 4, ywave = NTN >= 2 || w >= 4;
    const int nt0 = NTN >= 2 ? (w >> 2) * DN : 0;

    f4 h[NTN];  // rows j = 16w + 4lg + e, columns i = i0 + 16t + li
#pragma unroll
    for (int t = 0; t < NTN; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 16 * w + 4 * lg + e, i = i0 + 16 * t + li;
            h[t][e] = sr.s0 ? sr.s0[(head * D + i) * D + j] : 0.f;
        }
    auto fetch = [&](FwdFrags<DN> &f, int c) {
        const size_t ci = head * a.NC + c;
        const int t0 = c * C, n = min(C, T - t0), r = mrow + li;
        const bfr *wb = a.w.Wb + ci * C * D + frag_off<D>(mrow, 0) + 8 * l;
        const bfr *pb = a.w.Pb + ci * 2 * C * C + frag_off<C>(mrow, 0) + 8 * l;
        const bfr *kt = a.w.KTb + ci * D * C + frag_off<C>(16 * w, 0) + 8 * l;
        const bfr *qb = static_cast<const bfr *>(a.q) + (((size_t)b * a.Ts + t0 + r) * a.Hk + hk) * D + 8 * lg;
        const bfr *qg = VG ? a.w.QGb + ci * C * D + frag_off<D>(mrow, 0) + 8 * l : nullptr;
        // W and U in the waves that form Delta, Q and P in the waves that form y
        if (dwave) {
#pragma unroll
            for (int k = 0; k < 4; ++k) f.W[k] = ld_frag(wb + FRAG_BLOCK * k);
        }
        if (ywave) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (VG) f.Q[k] = ld_frag(qg + FRAG_BLOCK * k);
                else f.Q[k] = r < n ? ld_frag(qb + 32 * k) : zero_frag();
            }
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                f.P[k] = ld_frag(pb + FRAG_BLOCK * k);
                f.P[2 + k] = ld_frag(pb + C * C + FRAG_BLOCK * k);
            }
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) f.K[k] = ld_frag(kt + FRAG_BLOCK * k);
        if (dwave) {
#pragma unroll
            for (int t = 0; t < DN; ++t) {
                const float4 x = *reinterpret_cast<const float4 *>(a.w.U + ci * C * D + acc_off(mrow + 4 * lg, i0 + 16 * (nt0 + t) + li));
                f.U[t][0] = x.x; f.U[t][1] = x.y; f.U[t][2] = x.z; f.U[t][3] = x.w;
            }
        }
        if constexpr (VG) f.gc = *reinterpret_cast<const float4 *>(a.w.Gv + (ci * C + C - 1) * D + 16 * w + 4 * lg);
        else f.g = tid < C ? a.w.G[ci * C + tid] : 0.0;
    };
    // The chunk loop is unrolled by two over ping-pong fragment buffers: no register copy of the prefetched
    // fragments, so the wait for them sits at their first use, one chunk step after the loads were issued.
    auto step = [&](const int c, FwdFrags<DN> &cur, FwdFrags<DN> &nxt) {
        const int t0 = c * C, n = min(C, T - t0);
        const size_t ci = head * a.NC + c;
        if (float *sp = snap_at<MODE>(a, c)) store_state_acc<NTN>(sp, h, head, i0, w, lg, li);
        // h -> LDS as the operand [i][j]; the chunk-entry state -> saved H ([j][i], bf16)
#pragma unroll
        for (int t = 0; t < NTN; ++t) {
            acc_T<true>(h[t], sHh, sHl, LH, 16 * w, 16 * t);
            if constexpr (kTiles) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    reinterpret_cast<bfr *>(a.w.H)[ci * D * D + (size_t)(16 * w + 4 * lg + e) * D + i0 + 16 * t + li] =
                        (bfr)bfbits(h[t][e]);
            }
        }
        float *const sGam = sGamBuf[c & 1];
        if (!VG && tid < C) sGam[tid] = __builtin_amdgcn_exp2f((float)(cur.g * 1.4426950408889634));  // v_exp_f32 on log2 units
        __syncthreads();
        if (c + 1 < ce) fetch(nxt, c + 1);
        // Delta = U - W h ; Yi = Q h
        f4 yi[DN];
#pragma unroll
        for (int t = 0; t < DN; ++t) yi[t] = zero4();
        f4 wh[DN];
#pragma unroll
        for (int t = 0; t < DN; ++t) wh[t] = zero4();
        if (dwave) mmar<D, DN>(wh, cur.W, nullptr, sHh, nullptr, LH, 16 * nt0);
        if (ywave) mmar<D, DN, false, true>(yi, cur.Q, nullptr, sHh, sHl, LH, 16 * nt0);
        if (dwave) {
#pragma unroll
            for (int t = 0; t < DN; ++t) {
                f4 dl;
#pragma unroll
                for (int e = 0; e < 4; ++e) dl[e] = cur.U[t][e] - wh[t][e];
                acc_T<true>(dl, sDh, sDl, LDd, mrow, 16 * (nt0 + t));
                if constexpr (kTiles) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        a.w.Dl[ci * C * D + (size_t)(mrow + 4 * lg + e) * D + i0 + 16 * (nt0 + t) + li] = dl[e];
                }
            }
        }
        __syncthreads();
        if (ywave && kOut) {
            // Y = diag(gamma) Q h + P Delta  (per-channel gates: the decays are inside the Q * exp(G) tile)
            if constexpr (!VG) {
#pragma unroll
                for (int t = 0; t < DN; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) yi[t][e] *= sGam[mrow + 4 * lg + e];
            }
            mmar<C, DN, true, true>(yi, cur.P, cur.P + 2, sDh, sDl, LDd, 16 * nt0);
            // the output dtype is tested once for the whole tile, not at every element
            auto store_y = [&](auto dtag) {
                using E = decltype(dtag);
#pragma unroll
                for (int t = 0; t < DN; ++t)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int r = mrow + 4 * lg + e;
                        const size_t o = (((size_t)b * a.Ts + t0 + r) * a.Hv + hv) * D + i0 + 16 * (nt0 + t) + li;
                        if (r >= n) continue;
                        if constexpr (std::is_same<E, float>::value) static_cast<float *>(a.y)[o] = yi[t][e];
                        else if constexpr (std::is_same<E, uint16_t>::value) static_cast<uint16_t *>(a.y)[o] = f32_to_bf16_cvt(yi[t][e]);
                        else store_from_f32(a.y, o, yi[t][e], a.out_dt);
                    }
            };
            if (a.out_dt == DT_BF16) store_y(uint16_t{});
            else if (a.out_dt == DT_F32) store_y(float{});
            else store_y(int{});
        }
        // h = gamma_C h + (K diag(gamma_C / gamma))^T Delta  (per-channel gates: row j decays by exp(G_C,j))
        if constexpr (VG) {
            const float gcr[4] = {cur.gc.x, cur.gc.y, cur.gc.z, cur.gc.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = __builtin_amdgcn_exp2f(gcr[e]);  // G_C in log2 units
#pragma unroll
                for (int t = 0; t < NTN; ++t) h[t][e] *= d;
            }
        } else {
            const float gC = sGam[C - 1];
#pragma unroll
            for (int t = 0; t < NTN; ++t) h[t] *= gC;
        }
        mmar<C, NTN>(h, cur.K, nullptr, sDh, nullptr, LDd, 0);
    };
    FwdFrags<DN> fa, fb;
    fetch(fa, cb);
    for (int c = cb; c < ce; c += 2) {
        step(c, fa, fb);
        if (c + 1 < ce) step(c + 1, fb, fa);
    }
    if (kOut && a.state_T) store_state_acc<NTN>(a.state_T, h, head, i0, w, lg, li);
}

// ---------------------------------------------------------------------------------------------- ck_prep (bf16)
//
// ck_prep_kernel for bf16 inputs, on bf16 operand tiles read as 16-byte MFMA fragments.  The scalings are folded
// into T so that the second operand of W and U is the exact bf16 input:
//   W = (T diag(beta gamma)) K,   U = (T diag(beta)) V   (the T-side operand rounded to bf16, hi / lo for U).
// LDS regions are time-shared so that two workgroups fit on a CU:
//   R_K  K [64][LK]                          -> W staging (bf16 [64][LK])
//   R_Q  Q [64][LK]  -> V^T [128][LT]        -> U staging (fp32, spans R_Q and R_A)
//   R_A  A fp32 [64][LDC] -> K^T [128][LT]
//   R_T  T fp32 [64][LDC]
constexpr int LK = D + 8, LT = C + 8;
constexpr int PR_K = 0;
constexpr int PR_Q = PR_K + C * LK * 2;
constexpr int PR_A = PR_Q + D * LT * 2;
constexpr int PR_T = PR_A + D * LT * 2;
constexpr int PR_END = PR_T + C * LDC * 4;
constexpr int LU = D + 4;
static_assert(C * LDC * 4 <= D * LT * 2, "A fits its region");
static_assert(C * LU * 4 + C * LK * 2 <= PR_T, "U and W staging below T");

__global__ __launch_bounds__(NTP, 2) void ck_prep_bf16_kernel(Args a) {
    __shared__ __align__(16) unsigned char pa[PR_END];
    __shared__ float scratch[3 * 256];
    __shared__ double sG[C], sG2[C];  // G and G log2(e)
    __shared__ float sB[C], sBG[C], sRc[C];
    bfr *const sK = reinterpret_cast<bfr *>(pa + PR_K);
    bfr *const sQ = reinterpret_cast<bfr *>(pa + PR_Q);
    bfr *const sVT = sQ;
    float *const sA = reinterpret_cast<float *>(pa + PR_A);
    bfr *const sKT = reinterpret_cast<bfr *>(pa + PR_A);
    float *const sT = reinterpret_cast<float *>(pa + PR_T);

    const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk), t0 = c * C, n = min(C, T - t0);
    const size_t ci = chunk_index(a, b, hv, c);
    const size_t qk0 = (((size_t)b * a.Ts + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * a.Ts + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;

    // V as 8-token x 2-channel blocks (one per thread) for the transposed tile, kept in registers until Q is dead
    static_assert((C / 8) * (D / 2) == NTP, "one V block per thread");
    const int vb = tid / (D / 2), vc = 2 * (tid - vb * (D / 2));
    // rows past n read row n - 1 and are zeroed after: no load sits under a branch
    uint32_t vr[8];
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
        const int s2 = 8 * vb + rr;
        const uint32_t x =
            *reinterpret_cast<const uint32_t *>(static_cast<const bfr *>(a.v) + v0 + min(s2, n - 1) * v_row + vc);
        vr[rr] = s2 < n ? x : 0u;
    }
    // K and Q rows (16-byte pieces) and the gates: every load of the phase is issued before the first LDS store
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
    const size_t gi = ((size_t)b * a.Ts + t0 + min(tid, n - 1)) * a.Hv + hv;
    const float b_ld = a.beta[gi], g_ld = a.g[gi];
    const float bt = tid < n ? b_ld : 0.f, graw = tid < n ? g_ld : 1.f;
#pragma unroll
    for (int p = 0; p < KPER; ++p) {
        const int pc = tid + p * NTP, r = pc / (D / 8), c8 = (pc - r * (D / 8)) * 8;
        *reinterpret_cast<uint4 *>(sK + r * LK + c8) = kr[p];
        *reinterpret_cast<uint4 *>(sQ + r * LK + c8) = qr[p];
    }
    if (tid < C) {
        // inclusive prefix sum of the log decays in fp64 across wave 0
        const float gl = tid < n ? gate_log(graw, a.gate) : 0.f;
        const double x = wave_prefix_sum((double)gl);
        sB[tid] = bt;
        sG[tid] = x;
        sG2[tid] = x * 1.4426950408889634;  // log2(e): Gam_rs = 2^(G2_r - G2_s) on v_exp_f32
        sBG[tid] = bt * expf((float)x);
        sRc[tid] = expf((float)(readlane_f64(x, 63) - x));  // gamma_C / gamma_r
    }
    __syncthreads();
    // (K diag(gamma_C / gamma))^T (threads 0-255, for the forward) and Q^T (threads 256-511, for the backward) as
    // global bf16 tiles [j][r]: 8-token x 4-channel blocks, 4 stores of 8 consecutive tokens
    {
        const bool isq = tid >= (C / 8) * (D / 4);
        const int blk = isq ? tid - (C / 8) * (D / 4) : tid;
        const int rb = blk / (D / 4), j0 = (blk - rb * (D / 4)) * 4;
        const bfr *src = isq ? sQ : sK;
        float v[8][4];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const int r = rb * 8 + rr;
            const uint2 x = *reinterpret_cast<const uint2 *>(src + r * LK + j0);
            const float sc = isq ? 1.f : sRc[r];
            v[rr][0] = bf2f(x.x & 0xffffu) * sc; v[rr][1] = bf2f(x.x >> 16) * sc;
            v[rr][2] = bf2f(x.y & 0xffffu) * sc; v[rr][3] = bf2f(x.y >> 16) * sc;
        }
        // Q^T depends on the key head only: the first value head of each key head writes it
        const int rep = a.Hv / a.Hk;
        bfr *dst = isq ? a.w.QTb + (((size_t)b * a.Hk + hk) * a.NC + c) * D * C : a.w.KTb + ci * D * C;
        if (!isq || (hv % rep == 0 && !a.fwd_only)) {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
                *reinterpret_cast<uint4 *>(dst + frag_off<C>(j0 + cc, rb * 8)) =
                    make_uint4(pk(v[0][cc], v[1][cc]), pk(v[2][cc], v[3][cc]), pk(v[4][cc], v[5][cc]), pk(v[6][cc], v[7][cc]));
        }
    }
    // K K^T (waves 0-3) -> A = strict_lower(diag(beta) K K^T * Gam); Q K^T (waves 4-7) -> P = lower(Q K^T * Gam)
    // P hi / lo are staged in the T region (T is written only by the inverse, after the next barrier) and go out
    // in 16-byte stores; tiles above the diagonal (16t > r) are zero without an exponential.
    bfr *const sPb = reinterpret_cast<bfr *>(sT);  // [2][C][C]
    static_assert(2 * C * C * 2 <= C * LDC * 4, "P hi / lo fit the T region");
    {
        const int rb = w & 3, r0 = 16 * rb;
        const bool isq = w >= 4;
        f4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = zero4();
        mmab<D, 4>(acc, isq ? sQ : sK, nullptr, LK, r0, sK, nullptr, LK, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t ph[4], pl[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // branch-free: the exponential is formed in every lane and selected (above the diagonal it may
                // overflow; it is not used there)
                const int r = r0 + 4 * lg + e, s2 = 16 * t + li;
                const float ex = __builtin_amdgcn_exp2f((float)(sG2[r] - sG2[s2]));
                const float gam = t <= rb && s2 <= r ? ex : 0.f;
                if (isq) {
                    const float pv = acc[t][e] * gam;
                    ph[e] = bfbits(pv);
                    pl[e] = bfbits(pv - bf2f(ph[e]));
                    sPb[r * C + s2] = (bfr)ph[e];
                    sPb[C * C + r * C + s2] = (bfr)pl[e];
                } else {
                    sA[r * LDC + s2] = s2 < r ? sB[r] * acc[t][e] * gam : 0.f;
                }
            }
            if (isq && !a.fwd_only) {
                // P^T [s][r]: this lane's four consecutive r of column s = 16t + li
                bfr *pt = a.w.PTb + ci * 2 * C * C + frag_off<C>(16 * t + li, r0 + 4 * lg);
                *reinterpret_cast<uint2 *>(pt) = make_uint2(ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16));
                *reinterpret_cast<uint2 *>(pt + C * C) = make_uint2(pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16));
            }
        }
    }
    __syncthreads();  // Q read: its region takes V^T; P staged
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        uint32_t x[8];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) x[rr] = cc ? vr[rr] >> 16 : vr[rr] & 0xffffu;
        *reinterpret_cast<uint4 *>(sVT + (vc + cc) * LT + 8 * vb) =
            make_uint4(x[0] | (x[1] << 16), x[2] | (x[3] << 16), x[4] | (x[5] << 16), x[6] | (x[7] << 16));
    }
    for (int i = tid; i < 2 * C * C / 8; i += NTP) {  // P hi / lo out, in fragment order
        const int pl = i / (C * C / 8), e0 = 8 * i - pl * C * C, m = e0 / C;
        *reinterpret_cast<uint4 *>(a.w.Pb + ci * 2 * C * C + pl * C * C + frag_off<C>(m, e0 - m * C)) =
            *reinterpret_cast<const uint4 *>(sPb + 8 * i);
    }
    __syncthreads();  // P read out of the T region
    unit_lower_inverse<NTP>(sA, sT, scratch);  // ends with a barrier: A is dead
    // K^T [j][s] (exact) in the A region
    if (tid < (C / 8) * (D / 4)) {
        const int rb = tid / (D / 4), j0 = (tid - rb * (D / 4)) * 4;
        uint32_t x[8][2];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const uint2 y = *reinterpret_cast<const uint2 *>(sK + (rb * 8 + rr) * LK + j0);
            x[rr][0] = y.x;
            x[rr][1] = y.y;
        }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const int hw = cc >> 1, sh = (cc & 1) * 16;
            uint32_t e8[8];
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) e8[rr] = (x[rr][hw] >> sh) & 0xffffu;
            *reinterpret_cast<uint4 *>(sKT + (j0 + cc) * LT + rb * 8) =
                make_uint4(e8[0] | (e8[1] << 16), e8[2] | (e8[3] << 16), e8[4] | (e8[5] << 16), e8[6] | (e8[7] << 16));
        }
    }
    __syncthreads();
    // W = (T diag(beta gamma)) K (waves 0-3), U = (T diag(beta)) V (waves 4-7): 16-row strips of 8 tiles, the
    // T-side fragments built from fp32 T in registers
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
        const float *scl = (isu ? sB : sBG) + 32 * k + 8 * lg;
        bf8 ah, al;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float y = xv[i] * scl[i];
            ah[i] = (__bf16)y;
            al[i] = (__bf16)(y - (float)ah[i]);
        }
        const bfr *bt = isu ? sVT : sKT;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const bf8 y = frag(bt, LT, 16 * t, 32 * k);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, y, acc[t], 0, 0, 0);
            if (isu) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, y, acc[t], 0, 0, 0);
        }
    }
    __syncthreads();  // K, V^T, K^T read: their regions stage U (fp32) and W (bf16)
    float *const sU = reinterpret_cast<float *>(pa);
    bfr *const sW = reinterpret_cast<bfr *>(pa + C * LU * 4);
    if (isu) {
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) sU[(r0 + 4 * lg + e) * LU + 16 * t + li] = acc[t][e];
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            uint32_t wb[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wb[e] = bfbits(acc[t][e]);
                sW[(r0 + 4 * lg + e) * LK + 16 * t + li] = (bfr)wb[e];
            }
            // -W^T [j][r]; bf16 negation flips the sign bit
            if (!a.fwd_only) {
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
            make_float4(sU[rw * LU + cl], sU[(rw + 1) * LU + cl], sU[(rw + 2) * LU + cl], sU[(rw + 3) * LU + cl]);
    }
    for (int i = tid; i < C * D / 8; i += NTP) {  // W bf16 in fragment order
        const int r = i / (D / 8), c8 = (i - r * (D / 8)) * 8;
        *reinterpret_cast<uint4 *>(a.w.Wb + ci * C * D + frag_off<D>(r, c8)) = *reinterpret_cast<const uint4 *>(sW + r * LK + c8);
    }
    if (!a.fwd_only) {
        // T^T as bf16 hi and lo planes in fragment order, the A operand of TdD = T^T dDelta in ck_bwd_seq_bf16: the
        // 16-byte unit (s, r8) holds T^T[s][r8 .. r8 + 7] = T[r8 .. r8 + 7][s]; consecutive threads take consecutive s
        static_assert(C * C / 8 == NTP, "one unit per thread");
        bfr *const tb = reinterpret_cast<bfr *>(a.w.T) + ci * 2 * C * C;
        const int s = tid % C, r8 = (tid / C) * 8;
        float x[8];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) x[rr] = sT[(r8 + rr) * LDC + s];
        uint4 h, l;
        pk2(x[0], x[1], h.x, l.x);
        pk2(x[2], x[3], h.y, l.y);
        pk2(x[4], x[5], h.z, l.z);
        pk2(x[6], x[7], h.w, l.w);
        *reinterpret_cast<uint4 *>(tb + frag_off<C>(s, r8)) = h;
        *reinterpret_cast<uint4 *>(tb + C * C + frag_off<C>(s, r8)) = l;
    }
    if (tid < C) a.w.G[ci * C + tid] = sG[tid];
}

// ---------------------------------------------------------------------------------------------- ck_bwd_seq (bf16)
//
// Reverse over chunks like ck_bwd_seq_kernel, for bf16 inputs.  Per chunk, with dh' the adjoint of the chunk's
// exit state (this workgroup's value slice, in MFMA accumulators):
//   dDelta = diag(rc) K dh' + P^T dY,   dh = gamma_C dh' + Q^T diag(gamma) dY - W^T dDelta,
// and it saves TdD = T^T dDelta (fp32 [C][D]), the only form in which ck_bwd_local_bf16 needs T and dDelta.
// The A operands (K straight from the input, P^T hi / lo, Q^T and -W^T written by ck_prep) are read as MFMA
// fragments from global memory into registers one chunk ahead, with the chunk's dY slice; LDS carries what the
// waves exchange: dh' as the operand [i][j] (hi / lo), dY^T, (diag(gamma) dY)^T (hi / lo) and dDelta^T (hi / lo),
// and T^T (hi / lo, fragment order), whose 32 bytes per thread are loaded one chunk ahead and stored between the
// two barriers of the chunk that uses them.  Two barriers per chunk.
struct BwdFrags {
    bf8 K[4], PT[4], QT[2], WT[2];  // PT[0..1] hi, PT[2..3] lo; WT = -W^T
    double g;
    float4 gc;  // per-channel gates: G_C of this lane's four state rows
};

// VG: one decay per key channel (gdn_chunk_vg.hip wrote the tiles): dDelta = (K * exp(G_C - G)) dh' + P^T dY with that
// tile as the A operand, and dh = diag(exp(G_C)) dh' + (Q * exp(G))^T dY - W^T dDelta, (Q * exp(G))^T per value head.
template <int VS, bool DYF32, bool VG = false>
__global__ __launch_bounds__(NTS) void ck_bwd_seq_bf16_kernel(Args a) {
    constexpr int NTN = VS / 16, DN = NTN >= 2 ? NTN / 2 : 1;
    constexpr int LH = D + 8, LDd = C + 8;
    constexpr int NYB = (C / 8) * (VS / 2);  // 8-token x 2-column blocks of the dY slice
    static_assert(NYB <= NTS, "one dY block per thread");
    __shared__ __align__(16) bfr sHh[VS * LH];    // dh' [i][j], hi
    __shared__ __align__(16) bfr sHl[VS * LH];    // dh' lo
    __shared__ __align__(16) bfr sY[VS * LDd];    // dY^T [i][s]
    __shared__ __align__(16) bfr sYgh[VS * LDd];  // (diag(gamma) dY)^T hi
    __shared__ __align__(16) bfr sYgl[VS * LDd];  // (diag(gamma) dY)^T lo
    __shared__ __align__(16) bfr sDd[VS * LDd];   // dDelta^T [i][r], hi
    __shared__ __align__(16) bfr sDdl[VS * LDd];  // dDelta^T lo
    __shared__ __align__(16) bfr sTT[2 * C * C];  // T^T hi, lo (fragment order)
    __shared__ float sGam[C], sRc[C];
    static_assert(2 * C * C / 8 == 2 * NTS, "two 16-byte pieces of T^T per thread");

    const SeqBlock sb = seq_block();
    const int i0 = sb.slice * VS, hv = sb.hv, b = sb.b;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk);
    const size_t head = (size_t)b * a.Hv + hv;
    const int mrow = 16 * (w & 3);
    const bool cwave = NTN >= 2 || w < 4;
    // with 16-wide slices waves 4-7 form the saved TdD after the barrier while waves 0-3 go on
    const bool twave = NTN >= 2 || w >= 4;
    const int nt0 = NTN >= 2 ? (w >> 2) * DN : 0;
    // this thread's block of the dY slice: tokens 8 yb .. 8 yb + 7, slice columns yc, yc + 1
    const bool ythr = tid < NYB;
    const int yb = tid / (VS / 2), yc = 2 * (tid - yb * (VS / 2));

    f4 dh[NTN];  // rows j = 16w + 4lg + e, columns i = i0 + 16t + li
#pragma unroll
    for (int t = 0; t < NTN; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 16 * w + 4 * lg + e, i = i0 + 16 * t + li;
            dh[t][e] = a.dstate_T ? a.dstate_T[(head * D + i) * D + j] : 0.f;
        }
    // this thread's two 16-byte pieces of the fragment-order T^T (hi | lo) of the chunk processed next
    uint4 ttr0, ttr1;  // two scalars, not an array: an array of them stays on the stack at VS = 16
    auto fetch_tt = [&](int c) {
        const uint4 *src = reinterpret_cast<const uint4 *>(reinterpret_cast<const bfr *>(a.w.T) +
                                                           (head * a.NC + c) * 2 * C * C);
        ttr0 = src[tid];
        ttr1 = src[tid + NTS];
    };
    using YRaw = typename std::conditional<DYF32, float2, uint32_t>::type;
    auto fetch = [&](BwdFrags &f, YRaw (&y)[8], int c) {
        const size_t ci = head * a.NC + c;
        const int t0 = c * C, n = min(C, T - t0), r = mrow + li;
        const bfr *kb = static_cast<const bfr *>(a.k) + (((size_t)b * a.Ts + t0 + r) * a.Hk + hk) * D + 8 * lg;
        const bfr *kd = VG ? a.w.KDb + ci * C * D + frag_off<D>(mrow, 0) + 8 * l : nullptr;
        const bfr *pt = a.w.PTb + ci * 2 * C * C + frag_off<C>(mrow, 0) + 8 * l;
        const bfr *qt = a.w.QTb + (VG ? ci : ((size_t)b * a.Hk + hk) * a.NC + c) * D * C + frag_off<C>(16 * w, 0) + 8 * l;
        const bfr *wt = a.w.nWTb + ci * D * C + frag_off<C>(16 * w, 0) + 8 * l;
        // K and P^T only in the waves that form dDelta (all of them when NTN >= 2)
        if (cwave) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (VG) f.K[k] = ld_frag(kd + FRAG_BLOCK * k);
                else f.K[k] = r < n ? ld_frag(kb + 32 * k) : zero_frag();
            }
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                f.PT[k] = ld_frag(pt + FRAG_BLOCK * k);
                f.PT[2 + k] = ld_frag(pt + C * C + FRAG_BLOCK * k);
            }
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            f.QT[k] = ld_frag(qt + FRAG_BLOCK * k);
            f.WT[k] = ld_frag(wt + FRAG_BLOCK * k);
        }
        if constexpr (VG) f.gc = *reinterpret_cast<const float4 *>(a.w.Gv + (ci * C + C - 1) * D + 16 * w + 4 * lg);
        else f.g = tid < C ? a.w.G[ci * C + tid] : 0.0;
        if (ythr) {
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                const int s2 = 8 * yb + rr;
                const size_t off = (((size_t)b * a.Ts + t0 + s2) * a.Hv + hv) * D + i0 + yc;
                if constexpr (DYF32)
                    y[rr] = s2 < n ? *reinterpret_cast<const float2 *>(static_cast<const float *>(a.dy) + off)
                                   : make_float2(0.f, 0.f);
                else
                    y[rr] = s2 < n ? *reinterpret_cast<const uint32_t *>(static_cast<const bfr *>(a.dy) + off) : 0u;
            }
        }
    };
    // unrolled by two over ping-pong fragment buffers, as in ck_fwd_bf16_kernel; both steps of a pair are
    // unconditional (a prefetch used only under a branch is sunk to its use by the compiler)
    YRaw yr[8];
    auto step = [&](const int c, BwdFrags &cur, BwdFrags &nxt) {
        const size_t ci = head * a.NC + c;
        // dh' -> LDS as the operand [i][j] (hi / lo) and -> the saved dH ([j][i], fp32)
#pragma unroll
        for (int t = 0; t < NTN; ++t) {
            acc_T<true>(dh[t], sHh, sHl, LH, 16 * w, 16 * t);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                reinterpret_cast<bfr *>(a.w.dH)[ci * D * D + (size_t)(16 * w + 4 * lg + e) * D + i0 + 16 * t + li] =
                    (bfr)bfbits(dh[t][e]);
        }
        // dY^T (exact for bf16 dY) and the gates
        float yv[8][2];
        if (ythr) {
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) {
                if constexpr (DYF32) {
                    yv[rr][0] = yr[rr].x;
                    yv[rr][1] = yr[rr].y;
                } else {
                    yv[rr][0] = bf2f(yr[rr] & 0xffffu);
                    yv[rr][1] = bf2f(yr[rr] >> 16);
                }
            }
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
                *reinterpret_cast<uint4 *>(sY + (yc + cc) * LDd + 8 * yb) =
                    make_uint4(pk(yv[0][cc], yv[1][cc]), pk(yv[2][cc], yv[3][cc]), pk(yv[4][cc], yv[5][cc]),
                               pk(yv[6][cc], yv[7][cc]));
        }
        if (!VG && tid < C) {  // wave 0 holds the chunk's cumulative log decays
            const double gl = readlane_f64(cur.g, C - 1);
            sGam[tid] = __builtin_amdgcn_exp2f((float)(cur.g * 1.4426950408889634));  // v_exp_f32 on log2 units
            sRc[tid] = __builtin_amdgcn_exp2f((float)((gl - cur.g) * 1.4426950408889634));
        }
        __syncthreads();
        const float gC = VG ? 1.f : sGam[C - 1];
        if (ythr) {
            float gm[8];  // per-channel gates: the decays are inside the (Q * exp(G))^T tile
#pragma unroll
            for (int rr = 0; rr < 8; ++rr) gm[rr] = VG ? 1.f : sGam[8 * yb + rr];
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                uint4 hi, lo;
                pk2(gm[0] * yv[0][cc], gm[1] * yv[1][cc], hi.x, lo.x);
                pk2(gm[2] * yv[2][cc], gm[3] * yv[3][cc], hi.y, lo.y);
                pk2(gm[4] * yv[4][cc], gm[5] * yv[5][cc], hi.z, lo.z);
                pk2(gm[6] * yv[6][cc], gm[7] * yv[7][cc], hi.w, lo.w);
                *reinterpret_cast<uint4 *>(sYgh + (yc + cc) * LDd + 8 * yb) = hi;
                *reinterpret_cast<uint4 *>(sYgl + (yc + cc) * LDd + 8 * yb) = lo;
            }
        }
        // T^T of this chunk -> LDS (read after the second barrier; the previous chunk's reads ended before the
        // first barrier of this one); the next chunk's pieces are loaded after the second barrier
        reinterpret_cast<uint4 *>(sTT)[tid] = ttr0;
        reinterpret_cast<uint4 *>(sTT)[tid + NTS] = ttr1;
        if (c > 0) fetch(nxt, yr, c - 1);
        // dDelta = diag(rc) K dh' + P^T dY
        if (cwave) {
            f4 kd[DN], pd[DN];
#pragma unroll
            for (int t = 0; t < DN; ++t) kd[t] = pd[t] = zero4();
            mmar<D, DN, false, true>(kd, cur.K, nullptr, sHh, sHl, LH, 16 * nt0);
            mmar<C, DN, true, false>(pd, cur.PT, cur.PT + 2, sY, nullptr, LDd, 16 * nt0);
#pragma unroll
            for (int t = 0; t < DN; ++t) {
                f4 dd;
#pragma unroll
                for (int e = 0; e < 4; ++e) dd[e] = (VG ? kd[t][e] : kd[t][e] * sRc[mrow + 4 * lg + e]) + pd[t][e];
                acc_T<true>(dd, sDd, sDdl, LDd, mrow, 16 * (nt0 + t));
            }
        }
        __syncthreads();
        if (c > 0) fetch_tt(c - 1);
        if (twave) {
            // saved TdD = T^T dDelta (T^T and dDelta split): rows s = mrow + 4 lg + e, this slice's columns
            f4 tdd[DN];
#pragma unroll
            for (int t = 0; t < DN; ++t) tdd[t] = zero4();
#pragma unroll
            for (int k = 0; k < C / 32; ++k) {
                const bf8 th = ld_frag(sTT + frag_off<C>(mrow, 32 * k) + 8 * l);
                const bf8 tl = ld_frag(sTT + C * C + frag_off<C>(mrow, 32 * k) + 8 * l);
#pragma unroll
                for (int t = 0; t < DN; ++t) {
                    const bf8 yh = frag(sDd, LDd, 16 * (nt0 + t), 32 * k), ylo = frag(sDdl, LDd, 16 * (nt0 + t), 32 * k);
                    tdd[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, yh, tdd[t], 0, 0, 0);
                    tdd[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tl, yh, tdd[t], 0, 0, 0);
                    tdd[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(th, ylo, tdd[t], 0, 0, 0);
                }
            }
            float *const td = a.w.dDl + ci * C * D;
#pragma unroll
            for (int t = 0; t < DN; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) td[(size_t)(mrow + 4 * lg + e) * D + i0 + 16 * (nt0 + t) + li] = tdd[t][e];
        }
        // dh = gamma_C dh' + Q^T diag(gamma) dY + (-W^T) dDelta  (per-channel gates: row j decays by exp(G_C,j))
        if constexpr (VG) {
            const float gcr[4] = {cur.gc.x, cur.gc.y, cur.gc.z, cur.gc.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = __builtin_amdgcn_exp2f(gcr[e]);  // G_C in log2 units
#pragma unroll
                for (int t = 0; t < NTN; ++t) dh[t][e] *= d;
            }
        } else {
#pragma unroll
            for (int t = 0; t < NTN; ++t) dh[t] *= gC;
        }
        mmar<C, NTN, false, true>(dh, cur.QT, nullptr, sYgh, sYgl, LDd, 0);
        mmar<C, NTN>(dh, cur.WT, nullptr, sDd, nullptr, LDd, 0);
    };
    BwdFrags fa, fb;
    fetch(fa, yr, a.NC - 1);
    fetch_tt(a.NC - 1);
    int c = a.NC - 1;
    for (; c > 0; c -= 2) {
        step(c, fa, fb);
        step(c - 1, fb, fa);
    }
    if (c == 0) step(0, fa, fb);
    if (a.dstate0) {
#pragma unroll
        for (int t = 0; t < NTN; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 16 * w + 4 * lg + e, i = i0 + 16 * t + li;
                a.dstate0[(head * D + i) * D + j] = dh[t][e];
            }
    }
}

}  // namespace ck

// ---------------------------------------------------------------------------------------------- host side

constexpr int CK_C = ck::C;
constexpr int CK_D = ck::D;

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

ChunkSizes chunk_sizes(int B, int T, int Hk, int Hv, bool bf16, bool bwd, int vgk) {
    static_assert(CK_C == kChunkC && CK_D == kChunkD, "chunk geometry");
    ChunkSizes s{};
    const size_t NC = (size_t)(T + CK_C - 1) / CK_C;
    const size_t n = (size_t)B * Hv * NC, nk = (size_t)B * Hk * NC;  // chunk-heads, chunk-key-heads
    const size_t cd = (size_t)CK_C * CK_D, cc = (size_t)CK_C * CK_C, dd = (size_t)CK_D * CK_D;
    size_t off = 0;
    auto put = [&](ChunkSizes::Buf &bf, size_t bytes) {
        bf.off = off;
        bf.size = bytes;
        off += al256(bytes);
    };
    const bool vg = vgk && bf16, vgd = vgk == 2 && bf16;
    put(s.G, vg ? 0 : n * CK_C * 8);
    put(s.U, n * cd * 4);
    put(s.H, bwd ? n * dd * (bf16 ? 2 : 4) : 0);
    put(s.Dl, bwd ? n * cd * 4 : 0);
    put(s.T, bwd ? n * cc * 4 : 0);            // fp32, or T^T as bf16 hi / lo planes
    put(s.P, bf16 ? 0 : n * cc * 4);
    put(s.W, bf16 ? 0 : n * cd * 4);
    put(s.Wb, bf16 ? n * cd * 2 : 0);
    put(s.KTb, bf16 ? n * cd * 2 : 0);
    put(s.Pb, bf16 ? n * 2 * cc * 2 : 0);
    put(s.PTb, bf16 && bwd ? n * 2 * cc * 2 : 0);
    put(s.QTb, bf16 && bwd ? (vg ? n : nk) * cd * 2 : 0);
    put(s.nWTb, bf16 && bwd ? n * cd * 2 : 0);
    put(s.Gv, vg ? n * cd * 4 : 0);
    put(s.QGb, vg ? n * cd * 2 : 0);
    put(s.KDb, vg && bwd ? n * cd * 2 : 0);
    s.saved = off;
    off = 0;
    put(s.dH, n * dd * (bf16 ? 2 : 4));
    put(s.dDl, n * cd * 4);                    // fp32 dDelta, or TdD = T^T dDelta (bf16 set)
    // the bf16 set with one gate per head keeps its whole running dq | dk sum in registers (NQR of four pieces)
    put(s.part, bf16 && !vg && ck::NQR == 4 ? 0 : (size_t)B * T * (bf16 ? Hk : Hv) * 2 * CK_D * 4);
    put(s.vgd, vgd ? n * ck::VGD_FLOATS * 4 : 0);
    s.work = off;
    return s;
}

static ck::Args make_args(const ChunkCall &cc) {
    ck::Args a{};
    a.q = cc.q; a.k = cc.k; a.v = cc.v; a.g = cc.g; a.beta = cc.beta; a.state0 = cc.state0;
    a.dy = cc.dy; a.dstate_T = cc.dstate_T; a.y = cc.y; a.dq = cc.dq; a.dk = cc.dk; a.dv = cc.dv;
    a.state_T = cc.state_T;
    a.dg = cc.dg; a.dbeta = cc.dbeta; a.dstate0 = cc.dstate0;
    const bool bf16 = cc.in_dt == DT_BF16;
    const ChunkSizes s = chunk_sizes(cc.B, cc.T, cc.Hk, cc.Hv, bf16, !cc.fwd_only, vg_kind(cc.gate));
    char *sv = static_cast<char *>(cc.tiles);
    auto at = [&](const ChunkSizes::Buf &bf) -> void * { return bf.size ? sv + bf.off : nullptr; };
    a.w.H = static_cast<float *>(at(s.H));
    a.w.G = static_cast<double *>(at(s.G));
    a.w.T = static_cast<float *>(at(s.T));
    a.w.P = static_cast<float *>(at(s.P));
    a.w.W = static_cast<float *>(at(s.W));
    a.w.U = static_cast<float *>(at(s.U));
    a.w.Dl = static_cast<float *>(at(s.Dl));
    a.w.Wb = static_cast<unsigned short *>(at(s.Wb));
    a.w.KTb = static_cast<unsigned short *>(at(s.KTb));
    a.w.Pb = static_cast<unsigned short *>(at(s.Pb));
    a.w.PTb = static_cast<unsigned short *>(at(s.PTb));
    a.w.QTb = static_cast<unsigned short *>(at(s.QTb));
    a.w.nWTb = static_cast<unsigned short *>(at(s.nWTb));
    a.w.Gv = static_cast<float *>(at(s.Gv));
    a.w.QGb = static_cast<unsigned short *>(at(s.QGb));
    a.w.KDb = static_cast<unsigned short *>(at(s.KDb));
    if (cc.work) {
        char *wk = static_cast<char *>(cc.work);
        a.w.dH = reinterpret_cast<float *>(wk + s.dH.off);
        a.w.dDl = reinterpret_cast<float *>(wk + s.dDl.off);
        a.w.part = reinterpret_cast<float *>(wk + s.part.off);
        a.w.vgd = s.vgd.size ? reinterpret_cast<float *>(wk + s.vgd.off) : nullptr;
    }
    a.B = cc.B; a.T = cc.T; a.Ts = cc.Ts; a.Hk = cc.Hk; a.Hv = cc.Hv; a.NC = (cc.T + CK_C - 1) / CK_C;
    a.in_dt = cc.in_dt; a.out_dt = cc.out_dt; a.dy_dt = cc.dy_dt; a.grad_dt = cc.grad_dt; a.gate = cc.gate;
    a.snap = cc.snap; a.wc = cc.wc; a.win0 = cc.win0; a.recompute = cc.recompute; a.fwd_only = cc.fwd_only;
    return a;
}

// Value-slice width of the sequential kernels: the widest slice that still gives about one workgroup per CU
// (256 CUs), so fewer workgroups re-read the chunk's shared W / Q / K / P tiles.
static int slice_width(int heads) { return heads >= 128 ? 64 : heads >= 64 ? 32 : 16; }

// Workgroups along grid.z of the sequential kernels: the sequences, times the windows when they run side by side.
static int seq_z(const ck::Args &a) { return a.recompute ? a.B * ((a.NC + a.wc - 1) / a.wc) : a.B; }

// fp32 throughout: the fp32 set's kernels with the dtypes fixed at compile time
static bool all_f32(const ck::Args &a) {
    return a.in_dt == DT_F32 && a.dy_dt == DT_F32 && a.out_dt == DT_F32 && a.grad_dt == DT_F32;
}

// MT: the kernel set, 0 fp32 (fp32 / fp16 inputs), 1 bf16, 2 bf16 with one decay per key channel
template <int MT, int VS, int MODE>
static void fwd_launch(const ck::Args &a, hipStream_t st, dim3 grid) {
    if constexpr (MT == 2) hipLaunchKernelGGL((ck::ck_fwd_bf16_kernel<VS, MODE, true>), grid, dim3(ck::NTS), 0, st, a);
    else if constexpr (MT == 1) hipLaunchKernelGGL((ck::ck_fwd_bf16_kernel<VS, MODE>), grid, dim3(ck::NTS), 0, st, a);
    else if (all_f32(a)) hipLaunchKernelGGL((ck::ck_fwd_kernel<VS, MODE, true>), grid, dim3(ck::NTS), 0, st, a);
    else hipLaunchKernelGGL((ck::ck_fwd_kernel<VS, MODE, false>), grid, dim3(ck::NTS), 0, st, a);
}

template <int MT, int VS>
static void seq_launch(const ck::Args &a, hipStream_t st, bool fwd) {
    const dim3 grid(CK_D / VS, a.Hv, seq_z(a));
    if (fwd) {
        if (a.recompute) fwd_launch<MT, VS, ck::FWD_RECOMPUTE>(a, st, grid);
        else if (a.fwd_only) fwd_launch<MT, VS, ck::FWD_ONLY>(a, st, grid);
        else fwd_launch<MT, VS, ck::FWD_TRAIN>(a, st, grid);
    } else if constexpr (MT >= 1) {
        constexpr bool VG = MT == 2;
        if (a.dy_dt == DT_F32)
            hipLaunchKernelGGL((ck::ck_bwd_seq_bf16_kernel<VS, true, VG>), grid, dim3(ck::NTS), 0, st, a);
        else
            hipLaunchKernelGGL((ck::ck_bwd_seq_bf16_kernel<VS, false, VG>), grid, dim3(ck::NTS), 0, st, a);
    } else {
        if (all_f32(a)) hipLaunchKernelGGL((ck::ck_bwd_seq_kernel<VS, true>), grid, dim3(ck::NTS), 0, st, a);
        else hipLaunchKernelGGL((ck::ck_bwd_seq_kernel<VS, false>), grid, dim3(ck::NTS), 0, st, a);
    }
}

template <int MT>
static void seq_dispatch(const ck::Args &a, hipStream_t st, bool fwd) {
    switch (slice_width(seq_z(a) * a.Hv)) {
        case 64: seq_launch<MT, 64>(a, st, fwd); break;
        case 32: seq_launch<MT, 32>(a, st, fwd); break;
        default: seq_launch<MT, 16>(a, st, fwd); break;
    }
}

template <int MT>
static void ck_fwd_launch(const ck::Args &a, hipStream_t st, const char *stage) {
    if (stage[0] == 'p' && MT == 2)
        ck::launch_vg_prep(a, st);
    else if (stage[0] == 'p' && MT == 1)
        hipLaunchKernelGGL(ck::ck_prep_bf16_kernel, dim3(a.NC, a.Hv, a.B), dim3(ck::NTP), 0, st, a);
    else if (stage[0] == 'p' && all_f32(a))
        hipLaunchKernelGGL(ck::ck_prep_kernel<true>, dim3(a.NC, a.Hv, a.B), dim3(ck::NTP), 0, st, a);
    else if (stage[0] == 'p')
        hipLaunchKernelGGL(ck::ck_prep_kernel<false>, dim3(a.NC, a.Hv, a.B), dim3(ck::NTP), 0, st, a);
    else
        seq_dispatch<MT>(a, st, true);
}

template <int MT>
static void ck_bwd_launch(const ck::Args &a, hipStream_t st, const char *stage) {
    if (stage[0] == 's') {
        seq_dispatch<MT>(a, st, false);
    } else if (stage[0] == 'd') {
        if constexpr (MT == 2) ck::launch_vg_dg(a, st);
    } else if constexpr (MT == 2) {
        ck::launch_vg_local(a, st);
    } else if constexpr (MT == 1) {
        if (a.dy_dt == DT_F32)
            hipLaunchKernelGGL(ck::ck_bwd_local_bf16_kernel<true>, dim3(a.NC, a.Hk, a.B), dim3(ck::NTB), 0, st, a);
        else
            hipLaunchKernelGGL(ck::ck_bwd_local_bf16_kernel<false>, dim3(a.NC, a.Hk, a.B), dim3(ck::NTB), 0, st, a);
    }
    else if (all_f32(a))
        hipLaunchKernelGGL(ck::ck_bwd_local_kernel<true>, dim3(a.NC, a.Hk, a.B), dim3(ck::NTB), 0, st, a);
    else
        hipLaunchKernelGGL(ck::ck_bwd_local_kernel<false>, dim3(a.NC, a.Hk, a.B), dim3(ck::NTB), 0, st, a);
}

static int kernel_set(int in_dt, int gate) { return in_dt == DT_BF16 ? (gate_vec(gate) ? 2 : 1) : 0; }

bool chunk_vg_supported(int in_dt) { return in_dt == DT_BF16; }

void launch_chunk_stage(const ChunkCall &cc, const char *stage, hipStream_t st) {
    const ck::Args a = make_args(cc);
    const bool fwd = stage[0] == 'p' || stage[0] == 'f';
    switch (kernel_set(cc.in_dt, cc.gate)) {
        case 2: fwd ? ck_fwd_launch<2>(a, st, stage) : ck_bwd_launch<2>(a, st, stage); break;
        case 1: fwd ? ck_fwd_launch<1>(a, st, stage) : ck_bwd_launch<1>(a, st, stage); break;
        default: fwd ? ck_fwd_launch<0>(a, st, stage) : ck_bwd_launch<0>(a, st, stage); break;
    }
}

}  // namespace gdn
