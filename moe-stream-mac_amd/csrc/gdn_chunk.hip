// Chunked (WY / UT) form of the Gated DeltaNet forward and VJP for gfx950, chunk C = 64, Dk = Dv = D = 128.
//
// Per chunk of one head with entry state h = S^T ([Dk][Dv]), log decays g, G_r = sum_{u<=r} g_u (fp64),
// gamma = exp(G), Gam_rs = exp(G_r - G_s) for s <= r:
//   A = strict_lower(diag(beta) (K K^T) * Gam),  T = (I + A)^-1,  W = T diag(beta gamma) K,  U = T diag(beta) V
//   Delta = U - W h,  P = lower(Q K^T * Gam),  Y = diag(gamma) Q h + P Delta,
//   h' = gamma_C h + K^T diag(gamma_C / gamma) Delta
// which equals the token recurrence of engine/include/gdn.h:217-226 / tools/gdn_vjp.py:3-6 exactly in exact
// arithmetic.  The reverse pass is the adjoint of these matrix expressions (chunk-parallel except for the
// state adjoint, which runs backward over chunks like the forward state does).
//
// Kernels:
//   ck_prep      grid (NC, Hv, B): G, T (blocked 16x16 unit-lower inverse), W, U, P of one chunk.
//   ck_fwd       grid (D/VS, Hv, B): sequential over chunks; one value slice of h lives in MFMA accumulators.
//   ck_bwd_seq   grid (D/VS, Hv, B): reverse over chunks; the state adjoint dh and dDelta.
//   ck_bwd_local grid (NC, Hv, B): dq, dk (per value head), dv, dbeta, dg of one chunk.
// Matrix products run on MFMA: v_mfma_f32_16x16x4_f32 for fp32 inputs, v_mfma_f32_16x16x32_bf16 for bf16
// inputs (fp32 accumulation; the state stays fp32 in the accumulators).
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace ck {

constexpr int C = 64;
constexpr int D = 128;
constexpr int LD = D + 4;   // padded LDS row stride of [*][D] tiles
constexpr int LDC = C + 4;  // padded LDS row stride of [*][C] tiles
constexpr int NT = 256;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

// acc(16x16) += A(16 x K) * B(K x 16).  Element (r, c) of A is A[r*asr + c*asc]; element (k, n) of B is
// B[k*bsr + n*bsc]; both pointers are at the tile origin.  Accumulator element e of lane l is
// (row 4*(l/16) + e, column l%16).
// With bf16 MFMA (MT == 1) an operand flagged SA / SB is a computed fp32 value, not an exact bf16 input: it
// is split into hi = bf16(x) and lo = bf16(x - hi) and the product gets the extra hi*lo terms (about 16
// mantissa bits instead of 8).
template <int MT, int K, bool SA = false, bool SB = false>
__device__ __forceinline__ void mma16(f4 &acc, const float *A, int asr, int asc, const float *B, int bsr,
                                      int bsc) {
    const int l = threadIdx.x & 63, li = l & 15, lg = l >> 4;
    if constexpr (MT == 0) {
#pragma unroll 8
        for (int k0 = 0; k0 < K; k0 += 4) {
            const float av = A[li * asr + (k0 + lg) * asc];
            const float bv = B[(k0 + lg) * bsr + li * bsc];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
        }
    } else {
#pragma unroll 2
        for (int k0 = 0; k0 < K; k0 += 32) {
            bf8 ah, bh, al, bl;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = A[li * asr + (k0 + 8 * lg + i) * asc];
                const float y = B[(k0 + 8 * lg + i) * bsr + li * bsc];
                ah[i] = (__bf16)x;
                bh[i] = (__bf16)y;
                if constexpr (SA) al[i] = (__bf16)(x - (float)ah[i]);
                if constexpr (SB) bl[i] = (__bf16)(y - (float)bh[i]);
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
            if constexpr (SA) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
            if constexpr (SB) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
        }
    }
}

// Copy a [ROWS][COLS] tile (rows strided by src_stride elements, dtype dt) into LDS as fp32 with row stride
// lds_stride, multiplying row r by scale[r] when scale is given.  Rows >= n are zero.  Every load is 16 bytes
// and all of a thread's loads are issued before the first LDS store, so the tile costs one memory latency.
template <int ROWS, int COLS>
__device__ __forceinline__ void load_tile(float *dst, int lds_stride, const void *src, size_t src_stride, int n,
                                          int dt, const float *scale = nullptr) {
    const int tid = threadIdx.x;
    constexpr int BATCH = 8;  // 16-byte loads in flight per thread
    if (dt == DT_F32) {
        constexpr int VPR = COLS / 4;
        constexpr int PER = ROWS * VPR / NT;
        static_assert(PER * NT == ROWS * VPR, "tile must split evenly");
#pragma unroll
        for (int p0 = 0; p0 < PER; p0 += BATCH) {
            constexpr int NB = PER < BATCH ? PER : BATCH;
            float4 buf[NB];
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NT, r = v / VPR, c4 = (v - r * VPR) * 4;
                buf[p] = r < n ? *reinterpret_cast<const float4 *>(static_cast<const float *>(src) + r * src_stride + c4)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NT, r = v / VPR, c4 = (v - r * VPR) * 4;
                const float sc = scale ? scale[r] : 1.f;
                float *d = dst + r * lds_stride + c4;
                d[0] = buf[p].x * sc; d[1] = buf[p].y * sc; d[2] = buf[p].z * sc; d[3] = buf[p].w * sc;
            }
        }
    } else {
        constexpr int VPR = COLS / 8;
        constexpr int PER = ROWS * VPR / NT;
        static_assert(PER * NT == ROWS * VPR, "tile must split evenly");
#pragma unroll
        for (int p0 = 0; p0 < PER; p0 += BATCH) {
            constexpr int NB = PER < BATCH ? PER : BATCH;
            uint4 buf[NB];
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NT, r = v / VPR, c8 = (v - r * VPR) * 8;
                buf[p] = r < n ? *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(src) + r * src_stride + c8)
                               : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NT, r = v / VPR, c8 = (v - r * VPR) * 8;
                const float sc = scale ? scale[r] : 1.f;
                float *d = dst + r * lds_stride + c8;
                const uint32_t w4[4] = {buf[p].x, buf[p].y, buf[p].z, buf[p].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float lo, hi;
                    if (dt == DT_BF16) {
                        lo = __uint_as_float(w4[k] << 16);
                        hi = __uint_as_float(w4[k] & 0xffff0000u);
                    } else {
                        lo = __half2float(__ushort_as_half((unsigned short)(w4[k] & 0xffffu)));
                        hi = __half2float(__ushort_as_half((unsigned short)(w4[k] >> 16)));
                    }
                    d[2 * k] = lo * sc;
                    d[2 * k + 1] = hi * sc;
                }
            }
        }
    }
}

__device__ __forceinline__ const void *elem_ptr(const void *p, size_t idx, int dt) {
    return static_cast<const char *>(p) + idx * (dt == DT_F32 ? 4 : 2);
}

// Write the [D][D] state slab [i0, i0+VS) x [0, D) from its LDS copy sH ([j][ii], stride LV) to global in the
// reference layout S[i][j], one contiguous row of S per pass (coalesced along j).
template <int VS, int LV>
__device__ __forceinline__ void store_state_slice(float *dst, const float *sH, int i0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < VS * D / NT; ++p) {
        const int v = tid + p * NT, ii = v / D, j = v - ii * D;
        dst[(size_t)(i0 + ii) * D + j] = sH[j * LV + ii];
    }
}

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ float gate_log(float g, int gate) {
    if (gate == GATE_LOG) return g;
    // decay -> log decay; exp(-1e4) is exactly 0, and fp64 prefix sums stay exact at that magnitude
    return g > 0.f ? fmaxf(logf(g), -1e4f) : -1e4f;
}

struct Bufs {
    float *H;    // [B][Hv][NC][D][D] chunk-entry states, reference layout S[i][j]
    double *G;   // [B][Hv][NC][C]
    float *T;    // [B][Hv][NC][C][C]
    float *P;    // [B][Hv][NC][C][C]
    float *W;    // [B][Hv][NC][C][D]
    float *U;    // [B][Hv][NC][C][D]
    float *Dl;   // [B][Hv][NC][C][D]  Delta
    float *dH;   // [B][Hv][NC][D][D]  adjoint of each chunk's exit state
    float *dDl;  // [B][Hv][NC][C][D]  dDelta
    float *part; // [B][T][Hv][2][D]   dq | dk per value head
};

struct Args {
    const void *q, *k, *v;
    const float *g, *beta, *state0;
    const void *dy;
    const float *dstate_T;
    void *y, *dv;
    float *state_T, *dg, *dbeta, *dstate0;
    Bufs w;
    int B, T, Hk, Hv, NC, in_dt, out_dt, dy_dt, grad_dt, gate;
};

__device__ __forceinline__ size_t chunk_index(const Args &a, int b, int hv, int c) {
    return ((size_t)b * a.Hv + hv) * a.NC + c;
}

// (I + A)^-1 of a unit lower-triangular 64x64 matrix, A strictly lower in sA.  Diagonal 16x16 blocks by
// column-parallel forward substitution, then off-diagonal blocks by distance:
// T_ij = -T_ii sum_{u=j}^{i-1} A_iu T_uj.
__device__ void unit_lower_inverse(const float *sA, float *sT, float *scratch) {
    const int tid = threadIdx.x;
    for (int i = tid; i < C * C; i += NT) {
        const int r = i / C, s = i - r * C;
        if ((s >> 4) > (r >> 4)) sT[r * LDC + s] = 0.f;
    }
    if (tid < 64) {
        const int base = (tid >> 4) * 16, cc = tid & 15;
        float col[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            float s = (r == cc) ? 1.f : 0.f;
#pragma unroll
            for (int u = 0; u < r; ++u) s = fmaf(-sA[(base + r) * LDC + base + u], col[u], s);
            col[r] = s;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) sT[(base + r) * LDC + base + cc] = col[r];
    }
    __syncthreads();
    for (int d = 1; d < 4; ++d) {
        const int nb = 4 - d;
        for (int e = tid; e < nb * 256; e += NT) {
            const int blk = e >> 8, bi = blk + d, bj = blk, r = (e >> 4) & 15, cc = e & 15;
            float x = 0.f;
            for (int u = 16 * bj; u < 16 * bi; ++u) x = fmaf(sA[(16 * bi + r) * LDC + u], sT[u * LDC + 16 * bj + cc], x);
            scratch[e] = x;
        }
        __syncthreads();
        for (int e = tid; e < nb * 256; e += NT) {
            const int blk = e >> 8, bi = blk + d, bj = blk, r = (e >> 4) & 15, cc = e & 15;
            float t = 0.f;
#pragma unroll
            for (int v = 0; v < 16; ++v) t = fmaf(sT[(16 * bi + r) * LDC + 16 * bi + v], scratch[(blk << 8) + v * 16 + cc], t);
            sT[(16 * bi + r) * LDC + 16 * bj + cc] = -t;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------- ck_prep

template <int MT>
__global__ __launch_bounds__(NT) void ck_prep_kernel(Args a) {
    __shared__ __align__(16) float sK[C * LD];
    __shared__ __align__(16) float sX[C * LD];
    __shared__ __align__(16) float sA[C * LDC];
    __shared__ __align__(16) float sT[C * LDC];
    __shared__ float scratch[3 * 256];
    __shared__ double sG[C];
    __shared__ float sGl[C], sB[C], sGam[C];

    const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk), t0 = c * C, n = min(C, T - t0);
    const size_t ci = chunk_index(a, b, hv, c);

    const size_t qk0 = (((size_t)b * T + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * T + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;
    load_tile<C, D>(sK, LD, elem_ptr(a.k, qk0, a.in_dt), qk_row, n, a.in_dt);
    load_tile<C, D>(sX, LD, elem_ptr(a.q, qk0, a.in_dt), qk_row, n, a.in_dt);
    if (tid < C) {
        float bt = 0.f, gl = 0.f;
        if (tid < n) {
            const size_t gi = ((size_t)b * T + t0 + tid) * a.Hv + hv;
            bt = a.beta[gi];
            gl = gate_log(a.g[gi], a.gate);
        }
        sB[tid] = bt;
        sGl[tid] = gl;
    }
    __syncthreads();
    if (tid == 0) {
        double s = 0.0;
        for (int r = 0; r < C; ++r) {
            s += (double)sGl[r];
            sG[r] = s;
        }
    }
    __syncthreads();
    if (tid < C) sGam[tid] = expf((float)sG[tid]);
    // K K^T and Q K^T: wave w owns rows 16w..16w+15
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        f4 kk = zero4(), qk = zero4();
        mma16<MT, D>(kk, sK + 16 * w * LD, LD, 1, sK + 16 * nt * LD, 1, LD);
        mma16<MT, D>(qk, sX + 16 * w * LD, LD, 1, sK + 16 * nt * LD, 1, LD);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, s = 16 * nt + li;
            const float gam = s <= r ? expf((float)(sG[r] - sG[s])) : 0.f;
            sA[r * LDC + s] = s < r ? sB[r] * kk[e] * gam : 0.f;
            a.w.P[ci * C * C + r * C + s] = qk[e] * gam;
        }
    }
    __syncthreads();
    unit_lower_inverse(sA, sT, scratch);
    for (int i = tid; i < C * D; i += NT) {
        const int r = i / D, j = i - r * D;
        sK[r * LD + j] *= sB[r] * sGam[r];
    }
    load_tile<C, D>(sX, LD, elem_ptr(a.v, v0, a.in_dt), v_row, n, a.in_dt, sB);
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
        f4 wa = zero4(), ua = zero4();
        mma16<MT, C>(wa, sT + 16 * w * LDC, LDC, 1, sK + 16 * nt, LD, 1);
        mma16<MT, C, true, true>(ua, sT + 16 * w * LDC, LDC, 1, sX + 16 * nt, LD, 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, col = 16 * nt + li;
            a.w.W[ci * C * D + r * D + col] = wa[e];
            a.w.U[ci * C * D + r * D + col] = ua[e];
        }
    }
    for (int i = tid; i < C * C; i += NT) a.w.T[ci * C * C + i] = sT[(i / C) * LDC + (i % C)];
    if (tid < C) a.w.G[ci * C + tid] = sG[tid];
}

// ---------------------------------------------------------------------------------------------- ck_fwd

template <int MT, int VS>
__global__ __launch_bounds__(NT) void ck_fwd_kernel(Args a) {
    constexpr int LV = VS + 4;
    constexpr int NTN = VS / 16;
    __shared__ __align__(16) float sW[C * LD];  // W, then P (stride LDC)
    __shared__ __align__(16) float sQ[C * LD];  // gamma Q, then K diag(gamma_C / gamma)
    __shared__ __align__(16) float sU[C * LV];
    __shared__ __align__(16) float sH[D * LV];  // h slice, [j][i]
    __shared__ __align__(16) float sD[C * LV];  // Delta slice
    __shared__ double sG[C];
    __shared__ float sGam[C], sRc[C];

    const int i0 = blockIdx.x * VS, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk);
    const size_t head = (size_t)b * a.Hv + hv;

    f4 h[2][NTN];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 16 * (2 * w + mi) + 4 * lg + e, i = i0 + 16 * nt + li;
                h[mi][nt][e] = a.state0 ? a.state0[(head * D + i) * D + j] : 0.f;
            }
    for (int c = 0; c < a.NC; ++c) {
        const int t0 = c * C, n = min(C, T - t0);
        const size_t ci = head * a.NC + c;
        __syncthreads();
        const size_t qk0 = (((size_t)b * T + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
                for (int e = 0; e < 4; ++e) sH[(16 * (2 * w + mi) + 4 * lg + e) * LV + 16 * nt + li] = h[mi][nt][e];
        if (tid < C) sG[tid] = a.w.G[ci * C + tid];
        __syncthreads();
        if (tid < C) {
            sGam[tid] = expf((float)sG[tid]);
            sRc[tid] = expf((float)(sG[C - 1] - sG[tid]));
        }
        store_state_slice<VS, LV>(a.w.H + ci * D * D, sH, i0);
        load_tile<C, D>(sW, LD, a.w.W + ci * C * D, D, C, DT_F32);
        load_tile<C, VS>(sU, LV, a.w.U + ci * C * D + i0, D, C, DT_F32);
        __syncthreads();
        load_tile<C, D>(sQ, LD, elem_ptr(a.q, qk0, a.in_dt), qk_row, n, a.in_dt, sGam);
        __syncthreads();
        f4 yi[NTN];
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) {
            f4 wh = zero4();
            yi[nt] = zero4();
            mma16<MT, D>(wh, sW + 16 * w * LD, LD, 1, sH + 16 * nt, LV, 1);
            mma16<MT, D, true, true>(yi[nt], sQ + 16 * w * LD, LD, 1, sH + 16 * nt, LV, 1);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 16 * w + 4 * lg + e, ii = 16 * nt + li;
                const float dl = sU[r * LV + ii] - wh[e];
                sD[r * LV + ii] = dl;
                a.w.Dl[ci * C * D + r * D + i0 + ii] = dl;
            }
        }
        __syncthreads();
        load_tile<C, C>(sW, LDC, a.w.P + ci * C * C, C, C, DT_F32);
        load_tile<C, D>(sQ, LD, elem_ptr(a.k, qk0, a.in_dt), qk_row, n, a.in_dt, sRc);
        __syncthreads();
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) {
            mma16<MT, C, true, true>(yi[nt], sW + 16 * w * LDC, LDC, 1, sD + 16 * nt, LV, 1);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 16 * w + 4 * lg + e, ii = 16 * nt + li;
                if (r < n)
                    store_from_f32(a.y, (((size_t)b * T + t0 + r) * a.Hv + hv) * D + i0 + ii, yi[nt][e], a.out_dt);
            }
        }
        const float gC = sGam[C - 1];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nt = 0; nt < NTN; ++nt) {
                h[mi][nt] *= gC;
                mma16<MT, C>(h[mi][nt], sQ + 16 * (2 * w + mi), 1, LD, sD + 16 * nt, LV, 1);
            }
    }
    if (a.state_T) {
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = 16 * (2 * w + mi) + 4 * lg + e, i = i0 + 16 * nt + li;
                    a.state_T[(head * D + i) * D + j] = h[mi][nt][e];
                }
    }
}

// ---------------------------------------------------------------------------------------------- ck_bwd_seq

template <int MT, int VS>
__global__ __launch_bounds__(NT) void ck_bwd_seq_kernel(Args a) {
    constexpr int LV = VS + 4;
    constexpr int NTN = VS / 16;
    __shared__ __align__(16) float sW[C * LD];  // P (stride LDC), then W
    __shared__ __align__(16) float sQ[C * LD];  // K diag(gamma_C / gamma), then gamma Q
    __shared__ __align__(16) float sY[C * LV];  // dY slice
    __shared__ __align__(16) float sH[D * LV];  // dh slice, [j][i]
    __shared__ __align__(16) float sD[C * LV];  // dDelta slice
    __shared__ double sG[C];
    __shared__ float sGam[C], sRc[C];

    const int i0 = blockIdx.x * VS, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk);
    const size_t head = (size_t)b * a.Hv + hv;

    f4 dh[2][NTN];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = 16 * (2 * w + mi) + 4 * lg + e, i = i0 + 16 * nt + li;
                dh[mi][nt][e] = a.dstate_T ? a.dstate_T[(head * D + i) * D + j] : 0.f;
            }
    for (int c = a.NC - 1; c >= 0; --c) {
        const int t0 = c * C, n = min(C, T - t0);
        const size_t ci = head * a.NC + c;
        __syncthreads();
        const size_t qk0 = (((size_t)b * T + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
        const size_t v0 = (((size_t)b * T + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
                for (int e = 0; e < 4; ++e) sH[(16 * (2 * w + mi) + 4 * lg + e) * LV + 16 * nt + li] = dh[mi][nt][e];
        if (tid < C) sG[tid] = a.w.G[ci * C + tid];
        __syncthreads();
        if (tid < C) {
            sGam[tid] = expf((float)sG[tid]);
            sRc[tid] = expf((float)(sG[C - 1] - sG[tid]));
        }
        store_state_slice<VS, LV>(a.w.dH + ci * D * D, sH, i0);
        load_tile<C, C>(sW, LDC, a.w.P + ci * C * C, C, C, DT_F32);
        load_tile<C, VS>(sY, LV, elem_ptr(a.dy, v0 + i0, a.dy_dt), v_row, n, a.dy_dt);
        __syncthreads();
        load_tile<C, D>(sQ, LD, elem_ptr(a.k, qk0, a.in_dt), qk_row, n, a.in_dt, sRc);
        __syncthreads();
#pragma unroll
        for (int nt = 0; nt < NTN; ++nt) {
            f4 dd = zero4();
            mma16<MT, D, true, true>(dd, sQ + 16 * w * LD, LD, 1, sH + 16 * nt, LV, 1);
            mma16<MT, C, true, false>(dd, sW + 16 * w, 1, LDC, sY + 16 * nt, LV, 1);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 16 * w + 4 * lg + e, ii = 16 * nt + li;
                sD[r * LV + ii] = dd[e];
                a.w.dDl[ci * C * D + r * D + i0 + ii] = dd[e];
            }
        }
        __syncthreads();
        load_tile<C, D>(sW, LD, a.w.W + ci * C * D, D, C, DT_F32);
        load_tile<C, D>(sQ, LD, elem_ptr(a.q, qk0, a.in_dt), qk_row, n, a.in_dt, sGam);
        __syncthreads();
        const float gC = sGam[C - 1];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nt = 0; nt < NTN; ++nt) {
                f4 wd = zero4();
                dh[mi][nt] *= gC;
                mma16<MT, C, true, false>(dh[mi][nt], sQ + 16 * (2 * w + mi), 1, LD, sY + 16 * nt, LV, 1);
                mma16<MT, C>(wd, sW + 16 * (2 * w + mi), 1, LD, sD + 16 * nt, LV, 1);
                dh[mi][nt] -= wd;
            }
    }
    if (a.dstate0) {
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int nt = 0; nt < NTN; ++nt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = 16 * (2 * w + mi) + 4 * lg + e, i = i0 + 16 * nt + li;
                    a.dstate0[(head * D + i) * D + j] = dh[mi][nt][e];
                }
    }
}

// ---------------------------------------------------------------------------------------------- ck_bwd_local

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) x += __shfl_xor(x, m, 64);
    return x;
}

// dG bookkeeping.  Every term of the log-decay gradient depends on a difference G_r - G_s' of cumulative log
// decays (s' = -1 stands for the chunk start), so it is a "pair" term E[r][s'] that adds +E to dG_r and -E to
// dG_s'.  The gradient of the per-token log decay g_u is then the sum of the pair terms whose span straddles
// u:  dg_u = sum_{r >= u} sum_{s' < u} E[r][s'].  Summing only straddling terms (each carrying the factor
// exp(g_u)) keeps dg accurate for tiny decays, where a reverse cumulative sum of dG would cancel.
template <int MT>
__global__ __launch_bounds__(NT) void ck_bwd_local_kernel(Args a) {
    __shared__ __align__(16) float R1[D * LD];       // h / dh' ([i][j]); then K at R1, Q / dW at R1 + C*LD
    __shared__ __align__(16) float R2[C * LD];       // dY, then dDelta, then the pair matrix E
    __shared__ __align__(16) float RX[2 * C * LDC];  // V ([C][LD] fits), then R3 = RX (Y1), R4 = RX + C*LDC
    __shared__ __align__(16) float R5[C * LDC];      // T
    __shared__ double sG[C];
    __shared__ float sGam[C], sRc[C], sB[C], sEb[C], sT2[C], sDg[C];
    __shared__ float sLast[4];

    const int c = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    const int T = a.T, hk = hv / (a.Hv / a.Hk), t0 = c * C, n = min(C, T - t0);
    const size_t ci = chunk_index(a, b, hv, c);
    float *const sKm = R1;
    float *const sQm = R1 + C * LD;
    float *const R3 = RX;
    float *const R4 = RX + C * LDC;
    const float *Hc = a.w.H + ci * D * D;
    const float *dHc = a.w.dH + ci * D * D;
    const float *Dc = a.w.Dl + ci * C * D;
    const float *dDc = a.w.dDl + ci * C * D;
    // dW of this chunk is parked in its rows of the dq|dk output buffer until it is needed (rows >= n of dW
    // are zero: padded tokens have k = 0, so their dDelta vanishes)
    float *const dWpark = a.w.part + ((size_t)b * T + t0) * a.Hv * 2 * D + (size_t)hv * 2 * D;
    const size_t park_row = (size_t)a.Hv * 2 * D;

    // ---- phase 0: gates, dY, h
    if (tid < C) {
        sG[tid] = a.w.G[ci * C + tid];
        float bt = 0.f;
        if (tid < n) bt = a.beta[((size_t)b * T + t0 + tid) * a.Hv + hv];
        sB[tid] = bt;
    }
    const size_t qk0 = (((size_t)b * T + t0) * a.Hk + hk) * D, qk_row = (size_t)a.Hk * D;
    const size_t v0 = (((size_t)b * T + t0) * a.Hv + hv) * D, v_row = (size_t)a.Hv * D;
    load_tile<D, D>(R1, LD, Hc, D, D, DT_F32);
    load_tile<C, D>(R2, LD, elem_ptr(a.dy, v0, a.dy_dt), v_row, n, a.dy_dt);
    __syncthreads();
    if (tid < C) {
        sGam[tid] = expf((float)sG[tid]);
        sRc[tid] = expf((float)(sG[C - 1] - sG[tid]));
    }
    __syncthreads();
    const float gC = sGam[C - 1];
    float bnd[4] = {0.f, 0.f, 0.f, 0.f};   // pair terms (r, chunk start) of rows 16w+4lg+e, this lane's columns
    float rowB[4] = {0.f, 0.f, 0.f, 0.f};  // dbeta partials
    float lastp = 0.f;                     // pair (C-1, chunk start): gamma_C <dh', h>

    // <dh', h>: h is in R1, dh' streams from global in 16-byte loads, all issued up front
    {
        constexpr int PER = D * D / 4 / NT;
#pragma unroll
        for (int p0 = 0; p0 < PER; p0 += 8) {
            float4 dv4[8];
#pragma unroll
            for (int p = 0; p < 8; ++p) dv4[p] = reinterpret_cast<const float4 *>(dHc)[tid + (p0 + p) * NT];
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                const int v = tid + (p0 + p) * NT, i = v / (D / 4), j = (v - i * (D / 4)) * 4;
                const float *hh = R1 + i * LD + j;
                lastp += dv4[p].x * hh[0] + dv4[p].y * hh[1] + dv4[p].z * hh[2] + dv4[p].w * hh[3];
            }
        }
    }
    lastp *= gC;

    // ---- phase 1: dQ = diag(gamma) dY h^T ; dW = -dDelta h^T (parked in global)
    f4 dQ[8], dK[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
        f4 dw = zero4();
        dQ[nt] = zero4();
        mma16<MT, D>(dQ[nt], R2 + 16 * w * LD, LD, 1, R1 + 16 * nt, LD, 1);
        mma16<MT, D>(dw, dDc + 16 * w * D, D, 1, R1 + 16 * nt, LD, 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, j = 16 * nt + li;
            dQ[nt][e] *= sGam[r];
            if (r < n) dWpark[r * park_row + j] = -dw[e];
        }
    }
    __syncthreads();
    // ---- phase 2: dK = diag(gamma_C/gamma) Delta dh'^T ; dP = lower(dY Delta^T)
    load_tile<D, D>(R1, LD, dHc, D, D, DT_F32);
    __syncthreads();
    float tl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
        dK[nt] = zero4();
        mma16<MT, D, true, true>(dK[nt], Dc + 16 * w * D, D, 1, R1 + 16 * nt, LD, 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dK[nt][e] *= sRc[16 * w + 4 * lg + e];
        }
    }
    f4 dPG[4], Ep[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        f4 dp = zero4();
        mma16<MT, D, false, true>(dp, R2 + 16 * w * LD, LD, 1, Dc + 16 * nt * D, 1, D);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, s = 16 * nt + li;
            const float pv = s <= r ? dp[e] : 0.f;
            Ep[nt][e] = s < r ? pv * a.w.P[ci * C * C + r * C + s] : 0.f;
            dPG[nt][e] = s <= r ? pv * expf((float)(sG[r] - sG[s])) : 0.f;
        }
    }
    __syncthreads();
    // ---- phase 3: dQ += dPG K ; dK += dPG^T Q
    load_tile<C, D>(sKm, LD, elem_ptr(a.k, qk0, a.in_dt), qk_row, n, a.in_dt);
    load_tile<C, D>(sQm, LD, elem_ptr(a.q, qk0, a.in_dt), qk_row, n, a.in_dt);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) R4[(16 * w + 4 * lg + e) * LDC + 16 * nt + li] = dPG[nt][e];
    __syncthreads();
    // pair terms of the state-entry and state-exit factors, from the dQ / dK parts computed so far
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, j = 16 * nt + li;
            bnd[e] += sQm[r * LD + j] * dQ[nt][e];
            tl[e] += sKm[r * LD + j] * dK[nt][e];
        }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
        mma16<MT, C, true, false>(dQ[nt], R4 + 16 * w * LDC, LDC, 1, sKm + 16 * nt, LD, 1);
        mma16<MT, C, true, false>(dK[nt], R4 + 16 * w, 1, LDC, sQm + 16 * nt, LD, 1);
    }
    __syncthreads();
    // ---- phase 4: through T.  R1b <- dW, R2 <- dDelta, RX <- V, R5 <- T
    load_tile<C, D>(sQm, LD, dWpark, park_row, n, DT_F32);
    load_tile<C, D>(R2, LD, dDc, D, C, DT_F32);
    load_tile<C, D>(RX, LD, elem_ptr(a.v, v0, a.in_dt), v_row, n, a.in_dt);
    load_tile<C, C>(R5, LDC, a.w.T + ci * C * C, C, C, DT_F32);
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
        f4 tdw = zero4(), tdd = zero4();
        mma16<MT, C>(tdw, R5 + 16 * w, 1, LDC, sQm + 16 * nt, LD, 1);
        mma16<MT, C, true, true>(tdd, R5 + 16 * w, 1, LDC, R2 + 16 * nt, LD, 1);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, j = 16 * nt + li;
            const float bg = sB[r] * sGam[r];
            dK[nt][e] += bg * tdw[e];
            const float s4 = tdw[e] * sKm[r * LD + j];
            rowB[e] += sGam[r] * s4;
            bnd[e] += bg * s4;
            rowB[e] += RX[r * LD + j] * tdd[e];
            if (r < n)
                store_from_f32(a.dv, (((size_t)b * T + t0 + r) * a.Hv + hv) * D + j, sB[r] * tdd[e], a.grad_dt);
        }
    }
    f4 dT[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        f4 t1 = zero4(), t2 = zero4();
        mma16<MT, D>(t1, R2 + 16 * w * LD, LD, 1, RX + 16 * nt * LD, 1, LD);
        mma16<MT, D>(t2, sQm + 16 * w * LD, LD, 1, sKm + 16 * nt * LD, 1, LD);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int s = 16 * nt + li;
            dT[nt][e] = sB[s] * (t1[e] + sGam[s] * t2[e]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) R4[(16 * w + 4 * lg + e) * LDC + 16 * nt + li] = dT[nt][e];
    __syncthreads();
    // ---- phase 5: dA = -T^T dT T^T ; K K^T ; M = diag(beta) dA * Gam
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        f4 y1 = zero4();
        mma16<MT, C>(y1, R4 + 16 * w * LDC, LDC, 1, R5 + 16 * nt * LDC, 1, LDC);
#pragma unroll
        for (int e = 0; e < 4; ++e) R3[(16 * w + 4 * lg + e) * LDC + 16 * nt + li] = y1[e];
    }
    __syncthreads();
    f4 Mt[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        f4 da = zero4(), kk = zero4();
        mma16<MT, C>(da, R5 + 16 * w, 1, LDC, R3 + 16 * nt, LDC, 1);
        mma16<MT, D>(kk, sKm + 16 * w * LD, LD, 1, sKm + 16 * nt * LD, 1, LD);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, s = 16 * nt + li;
            const float gam = s < r ? expf((float)(sG[r] - sG[s])) : 0.f;
            const float dav = s < r ? -da[e] : 0.f;
            const float kg = kk[e] * gam;
            rowB[e] += dav * kg;
            Ep[nt][e] += dav * sB[r] * kg;
            Mt[nt][e] = sB[r] * dav * gam;
        }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) R4[(16 * w + 4 * lg + e) * LDC + 16 * nt + li] = Mt[nt][e];
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
        mma16<MT, C>(dK[nt], R4 + 16 * w * LDC, LDC, 1, sKm + 16 * nt, LD, 1);
        mma16<MT, C>(dK[nt], R4 + 16 * w, 1, LDC, sKm + 16 * nt, LD, 1);
    }
    // ---- phase 6: straddle sums for dg, dbeta, outputs.  R2 (dDelta) is free: E goes there.
    float *const sE = R2;
    lastp = wave_sum(lastp);
    if (l == 0) sLast[w] = lastp;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) sE[(16 * w + 4 * lg + e) * LDC + 16 * nt + li] = Ep[nt][e];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float bsum = row16_allreduce(bnd[e]);
        const float t2 = row16_allreduce(tl[e]);
        const float rbv = row16_allreduce(rowB[e]);
        const int r = 16 * w + 4 * lg + e;
        if (li == 0) {
            sEb[r] = bsum;
            sT2[r] = r < C - 1 ? t2 : 0.f;   // pair (C-1, r); r = C-1 contributes nothing
            if (r < n) a.dbeta[((size_t)b * T + t0 + r) * a.Hv + hv] = rbv;
        }
    }
    __syncthreads();
    if (tid < C) {
        // row prefix sums of E over s' = 0 .. r-1, in place
        float acc = 0.f;
        for (int s2 = 0; s2 < C; ++s2) {
            const float x = sE[tid * LDC + s2];
            sE[tid * LDC + s2] = acc;   // = sum_{s' < s2} E[tid][s']
            acc += s2 < tid ? x : 0.f;
        }
        if (tid == C - 1) sEb[tid] += sLast[0] + sLast[1] + sLast[2] + sLast[3];
    }
    __syncthreads();
    if (tid < C) {
        const int u = tid;
        float acc = 0.f;
        for (int r = u; r < C; ++r) acc += sE[r * LDC + u] + sEb[r];
        for (int s2 = 0; s2 < u; ++s2) acc += sT2[s2];
        sDg[u] = acc;
    }
    __syncthreads();
    if (tid < n) {
        const size_t gi = ((size_t)b * T + t0 + tid) * a.Hv + hv;
        float dgv = sDg[tid];
        if (a.gate == GATE_DECAY) {
            const float dec = a.g[gi];
            dgv = dec > 1e-30f ? dgv / dec : 0.f;
        }
        a.dg[gi] = dgv;
    }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 16 * w + 4 * lg + e, j = 16 * nt + li;
            if (r < n) {
                const size_t tok = ((size_t)b * T + t0 + r) * a.Hv + hv;
                a.w.part[tok * 2 * D + j] = dQ[nt][e];
                a.w.part[tok * 2 * D + D + j] = dK[nt][e];
            }
        }
}

}  // namespace ck

// ---------------------------------------------------------------------------------------------- host side

constexpr int CK_C = ck::C;
constexpr int CK_D = ck::D;

static size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

ChunkSizes chunk_sizes(int B, int T, int Hv) {
    ChunkSizes s{};
    const size_t NC = (size_t)(T + CK_C - 1) / CK_C;
    const size_t heads = (size_t)B * Hv;
    size_t off = 0;
    s.H = off; off += al256(heads * NC * CK_D * CK_D * 4);
    s.G = off; off += al256(heads * NC * CK_C * 8);
    s.T = off; off += al256(heads * NC * CK_C * CK_C * 4);
    s.P = off; off += al256(heads * NC * CK_C * CK_C * 4);
    s.W = off; off += al256(heads * NC * CK_C * CK_D * 4);
    s.U = off; off += al256(heads * NC * CK_C * CK_D * 4);
    s.Dl = off; off += al256(heads * NC * CK_C * CK_D * 4);
    s.saved = off;
    off = 0;
    s.dH = off; off += al256(heads * NC * CK_D * CK_D * 4);
    s.dDl = off; off += al256(heads * NC * CK_C * CK_D * 4);
    s.part = off; off += al256((size_t)B * T * Hv * 2 * CK_D * 4);
    s.work = off;
    return s;
}

static ck::Args make_args(const ChunkCall &cc) {
    ck::Args a{};
    a.q = cc.q; a.k = cc.k; a.v = cc.v; a.g = cc.g; a.beta = cc.beta; a.state0 = cc.state0;
    a.dy = cc.dy; a.dstate_T = cc.dstate_T; a.y = cc.y; a.dv = cc.dv; a.state_T = cc.state_T;
    a.dg = cc.dg; a.dbeta = cc.dbeta; a.dstate0 = cc.dstate0;
    const ChunkSizes s = chunk_sizes(cc.B, cc.T, cc.Hv);
    char *sv = static_cast<char *>(cc.saved);
    a.w.H = reinterpret_cast<float *>(sv + s.H);
    a.w.G = reinterpret_cast<double *>(sv + s.G);
    a.w.T = reinterpret_cast<float *>(sv + s.T);
    a.w.P = reinterpret_cast<float *>(sv + s.P);
    a.w.W = reinterpret_cast<float *>(sv + s.W);
    a.w.U = reinterpret_cast<float *>(sv + s.U);
    a.w.Dl = reinterpret_cast<float *>(sv + s.Dl);
    if (cc.work) {
        char *wk = static_cast<char *>(cc.work);
        a.w.dH = reinterpret_cast<float *>(wk + s.dH);
        a.w.dDl = reinterpret_cast<float *>(wk + s.dDl);
        a.w.part = reinterpret_cast<float *>(wk + s.part);
    }
    a.B = cc.B; a.T = cc.T; a.Hk = cc.Hk; a.Hv = cc.Hv; a.NC = (cc.T + CK_C - 1) / CK_C;
    a.in_dt = cc.in_dt; a.out_dt = cc.out_dt; a.dy_dt = cc.dy_dt; a.grad_dt = cc.grad_dt; a.gate = cc.gate;
    return a;
}

constexpr int CK_VS = 32;

template <int MT>
static void ck_fwd_launch(const ck::Args &a, hipStream_t st, const char *stage) {
    if (stage[0] == 'p')
        hipLaunchKernelGGL((ck::ck_prep_kernel<MT>), dim3(a.NC, a.Hv, a.B), dim3(ck::NT), 0, st, a);
    else
        hipLaunchKernelGGL((ck::ck_fwd_kernel<MT, CK_VS>), dim3(CK_D / CK_VS, a.Hv, a.B), dim3(ck::NT), 0, st, a);
}

template <int MT>
static void ck_bwd_launch(const ck::Args &a, hipStream_t st, const char *stage) {
    if (stage[0] == 's')
        hipLaunchKernelGGL((ck::ck_bwd_seq_kernel<MT, CK_VS>), dim3(CK_D / CK_VS, a.Hv, a.B), dim3(ck::NT), 0, st, a);
    else
        hipLaunchKernelGGL((ck::ck_bwd_local_kernel<MT>), dim3(a.NC, a.Hv, a.B), dim3(ck::NT), 0, st, a);
}

static int mma_kind(int in_dt) { return in_dt == DT_BF16 ? 1 : 0; }

void launch_chunk_stage(const ChunkCall &cc, const char *stage, hipStream_t st) {
    const ck::Args a = make_args(cc);
    const bool fwd = stage[0] == 'p' || stage[0] == 'f';
    if (fwd) {
        if (mma_kind(cc.in_dt)) ck_fwd_launch<1>(a, st, stage);
        else ck_fwd_launch<0>(a, st, stage);
    } else {
        if (mma_kind(cc.in_dt)) ck_bwd_launch<1>(a, st, stage);
        else ck_bwd_launch<0>(a, st, stage);
    }
}

}  // namespace gdn
