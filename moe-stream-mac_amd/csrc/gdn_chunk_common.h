// Device helpers and launch arguments shared by the chunked-form kernels (gdn_chunk.hip, gdn_chunk_vg.hip):
// tile geometry, the fp32 and bf16 MFMA tile helpers, the kernel arguments and their per-chunk buffers, and the
// blocked unit-lower-triangular inverse.
#pragma once

#include "gdn_common.h"
#include "gdn_internal.h"

#include <type_traits>

namespace gdn {
namespace ck {

constexpr int C = 64;
constexpr int D = 128;
constexpr int LD = D + 4;   // padded LDS row stride of [*][D] tiles
constexpr int LDC = C + 4;  // padded LDS row stride of [*][C] tiles
constexpr int NT = 256;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

// A 16-row strip of NTILES output tiles sharing one A operand, fp32 MFMA (v_mfma_f32_16x16x4_f32):
// acc[t] += A(16 x K) * B_t(K x 16), where B_t starts at B + t * btile.  Element (r, c) of A is A[r*asr + c*asc];
// element (k, n) of B_t is B_t[k*bsr + n*bsc].  Accumulator element e of lane l is (row 4*(l/16) + e, column l%16).
template <int K, int NTILES>
__device__ __forceinline__ void mma_strip(f4 (&acc)[NTILES], const float *A, int asr, int asc, const float *B,
                                          int bsr, int bsc, int btile, int l = threadIdx.x & 63) {
    const int li = l & 15, lg = l >> 4;
    if constexpr (NTILES == 1 && K % 8 == 0) {
        // one tile: even and odd k-steps on two accumulators, so two products are in flight instead of one
        // dependent chain of K / 4
        f4 odd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int k0 = 0; k0 < K; k0 += 8) {
            const float a0 = A[li * asr + (k0 + lg) * asc], a1 = A[li * asr + (k0 + 4 + lg) * asc];
            const float b0 = B[(k0 + lg) * bsr + li * bsc], b1 = B[(k0 + 4 + lg) * bsr + li * bsc];
            acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0], 0, 0, 0);
            odd = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, odd, 0, 0, 0);
        }
        acc[0] += odd;
    } else {
#pragma unroll 4
        for (int k0 = 0; k0 < K; k0 += 4) {
            const float av = A[li * asr + (k0 + lg) * asc];
#pragma unroll
            for (int t = 0; t < NTILES; ++t) {
                const float bv = B[t * btile + (k0 + lg) * bsr + li * bsc];
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[t], 0, 0, 0);
            }
        }
    }
}

// Copy a [ROWS][COLS] tile (rows strided by src_stride elements, dtype dt) into LDS as fp32 with row stride
// lds_stride, multiplying row r by scale[r] when scale is given.  Rows >= n are zero (n >= 1: they load row n - 1
// and select zero, so no load sits under a branch, where the compiler would wait for it).  Every load is 16 bytes
// and all of a thread's loads are issued before the first LDS store, so the tile costs one memory latency.
template <int ROWS, int COLS, int NTH = NT>
__device__ __forceinline__ void load_tile(float *dst, int lds_stride, const void *src, size_t src_stride, int n,
                                          int dt, const float *scale = nullptr, int tid = threadIdx.x) {
    constexpr int BATCH = 8;  // 16-byte loads in flight per thread
    if (dt == DT_F32) {
        constexpr int VPR = COLS / 4;
        constexpr int PER = ROWS * VPR / NTH;
        static_assert(PER * NTH == ROWS * VPR, "tile must split evenly");
#pragma unroll
        for (int p0 = 0; p0 < PER; p0 += BATCH) {
            constexpr int NB = PER < BATCH ? PER : BATCH;
            float4 buf[NB];
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NTH, r = v / VPR, c4 = (v - r * VPR) * 4;
                const float *row = static_cast<const float *>(src) + min(r, n - 1) * src_stride;
                const float4 x = *reinterpret_cast<const float4 *>(row + c4);
                buf[p] = r < n ? x : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NTH, r = v / VPR, c4 = (v - r * VPR) * 4;
                const float sc = scale ? scale[r] : 1.f;
                float *d = dst + r * lds_stride + c4;
                d[0] = buf[p].x * sc; d[1] = buf[p].y * sc; d[2] = buf[p].z * sc; d[3] = buf[p].w * sc;
            }
        }
    } else {
        constexpr int VPR = COLS / 8;
        constexpr int PER = ROWS * VPR / NTH;
        static_assert(PER * NTH == ROWS * VPR, "tile must split evenly");
#pragma unroll
        for (int p0 = 0; p0 < PER; p0 += BATCH) {
            constexpr int NB = PER < BATCH ? PER : BATCH;
            uint4 buf[NB];
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NTH, r = v / VPR, c8 = (v - r * VPR) * 8;
                const uint16_t *row = static_cast<const uint16_t *>(src) + min(r, n - 1) * src_stride;
                const uint4 x = *reinterpret_cast<const uint4 *>(row + c8);
                buf[p] = r < n ? x : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int p = 0; p < NB; ++p) {
                const int v = tid + (p0 + p) * NTH, r = v / VPR, c8 = (v - r * VPR) * 8;
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

// Register staging for prefetch: a [ROWS][COLS] tile fetched as raw 16-byte quads (fp32: 4 elements, 16-bit
// dtypes: 8), later written to LDS as fp32.  Rows >= n read as zero.
template <int ROWS, int COLS, int NTH>
struct TileRegs {
    static constexpr int TOTAL_F32 = ROWS * COLS / 4;
    static constexpr int MAXQ = (TOTAL_F32 + NTH - 1) / NTH;
    uint4 q[MAXQ];
};

template <int ROWS, int COLS, int NTH>
__device__ __forceinline__ void tile_fetch(TileRegs<ROWS, COLS, NTH> &R, const void *src, size_t src_stride, int n,
                                           int dt) {
    const int tid = threadIdx.x;
    const int epq = dt == DT_F32 ? 4 : 8;               // elements per quad
    const int vpr = COLS / epq, total = ROWS * vpr;
    const int esz = dt == DT_F32 ? 4 : 2;
#pragma unroll
    for (int p = 0; p < TileRegs<ROWS, COLS, NTH>::MAXQ; ++p) {
        const int v = tid + p * NTH, r = v / vpr, c = (v - r * vpr) * epq;
        R.q[p] = (v < total && r < n)
                     ? *reinterpret_cast<const uint4 *>(static_cast<const char *>(src) + (r * src_stride + c) * esz)
                     : make_uint4(0u, 0u, 0u, 0u);
    }
}

__device__ __forceinline__ void unpack16(uint32_t w, int dt, float &lo, float &hi) {
    if (dt == DT_BF16) {
        lo = __uint_as_float(w << 16);
        hi = __uint_as_float(w & 0xffff0000u);
    } else {
        lo = __half2float(__ushort_as_half((unsigned short)(w & 0xffffu)));
        hi = __half2float(__ushort_as_half((unsigned short)(w >> 16)));
    }
}

// Write a fetched tile to LDS (row stride lds_stride), row r multiplied by scale(r) when given.
template <int ROWS, int COLS, int NTH, typename Scale>
__device__ __forceinline__ void tile_store(float *dst, int lds_stride, const TileRegs<ROWS, COLS, NTH> &R, int dt,
                                           Scale scale) {
    const int tid = threadIdx.x;
    const int epq = dt == DT_F32 ? 4 : 8;
    const int vpr = COLS / epq, total = ROWS * vpr;
#pragma unroll
    for (int p = 0; p < TileRegs<ROWS, COLS, NTH>::MAXQ; ++p) {
        const int v = tid + p * NTH, r = v / vpr, c = (v - r * vpr) * epq;
        if (v < total) {
            const float sc = scale(r);
            float *d = dst + r * lds_stride + c;
            if (dt == DT_F32) {
                d[0] = __uint_as_float(R.q[p].x) * sc;
                d[1] = __uint_as_float(R.q[p].y) * sc;
                d[2] = __uint_as_float(R.q[p].z) * sc;
                d[3] = __uint_as_float(R.q[p].w) * sc;
            } else {
                const uint32_t w4[4] = {R.q[p].x, R.q[p].y, R.q[p].z, R.q[p].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float lo, hi;
                    unpack16(w4[k], dt, lo, hi);
                    d[2 * k] = lo * sc;
                    d[2 * k + 1] = hi * sc;
                }
            }
        }
    }
}

struct NoScale {
    __device__ float operator()(int) const { return 1.f; }
};

__device__ __forceinline__ const void *elem_ptr(const void *p, size_t idx, int dt) {
    return static_cast<const char *>(p) + idx * (dt == DT_F32 ? 4 : 2);
}

// Write the value slab [i0, i0+VS) of a [D][D] chunk state from its LDS copy sH ([j][ii], stride LV) to global
// as h = S^T, element (j, i) at dst[j * D + i]: the layout the backward reads as MFMA operands (rows j, the
// reduction index i contiguous).  Stores are coalesced along i.
template <int VS, int LV, int NTH>
__device__ __forceinline__ void store_state_slice(float *dst, const float *sH, int i0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < VS * D / NTH; ++p) {
        const int v = tid + p * NTH, j = v / VS, ii = v - j * VS;
        dst[(size_t)j * D + i0 + ii] = sH[j * LV + ii];
    }
}

__device__ __forceinline__ f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }

// The smallest decay the chunked form takes in the decay conventions: a smaller one, zero included, runs as 2^-64.
// The state then keeps 2^-64 of itself where a zero decay keeps none (far below the fp32 rounding of the other terms),
// and every pair term that straddles such a token carries that factor, so dg = dg_log / 2^-64 is the derivative
// with respect to the decay there instead of 0 / 0.
constexpr float kMinDecay = 5.42101086242752217e-20f;  // 2^-64
constexpr float kLogMinDecay = -44.3614195558365f;     // ln 2^-64

// The per-token log decay the chunked form accumulates.  A log decay of -inf (a zero decay) is taken as -1e4, whose
// exponential is exactly 0, so that differences of cumulative sums stay finite; NaN passes through.  No branch: a
// conditional logf made the compiler wait for every load in flight before each one.
__device__ __forceinline__ float gate_log(float g, int gate) {
    if (gate_in_log(gate)) return g < -1e4f ? -1e4f : g;
    const float l = logf(fmaxf(g, kMinDecay));  // logf(2^-64) = kLogMinDecay
    return g == g ? l : g;
}

// d/d(decay) from d/d(log decay) at the decay the chunked form ran with
__device__ __forceinline__ float dg_per_decay(float dg_log, float d) { return dg_log / fmaxf(d, kMinDecay); }

struct Bufs {
    float *H;    // [B][Hv][NC][D][D] chunk-entry states h = S^T, element (j, i) at [j][i] (bf16 bits in the bf16 path)
    double *G;   // [B][Hv][NC][C]
    float *T;    // [B][Hv][NC][C][C] (bf16 path: T^T as bf16 hi and lo planes [2][C][C] in fragment order, same space)
    float *P;    // [B][Hv][NC][C][C]
    float *W;    // [B][Hv][NC][C][D]
    float *U;    // [B][Hv][NC][C][D]
    float *Dl;   // [B][Hv][NC][C][D]  Delta
    float *dH;   // [B][Hv][NC][D][D]  adjoint of each chunk's exit state, [j][i] like H (bf16 in the bf16 path)
    float *dDl;  // [B][Hv][NC][C][D]  dDelta (bf16 path: TdD = T^T dDelta, fp32)
    float *part; // [B][T][Hv][2][D]   ck_bwd_local scratch: the running dq | dk sum of a key head (per-channel
                 // gates: in the rows [B][T][Hk][2][D]; fp32 set: in the slot of the key head's first value head, the
                 // other slots parking each value head's dW; the bf16 set with one gate per head keeps the sum in
                 // registers and has no part buffer)
    // bf16 operand tiles written by ck_prep for the bf16 sequential kernels (raw bf16 bits), each [M][K] tile in
    // fragment order (frag_off<K>); the bf16 set keeps U in accumulator order (acc_off)
    unsigned short *Wb;   // [B][Hv][NC][C][D]     W
    unsigned short *KTb;  // [B][Hv][NC][D][C]     (K diag(gamma_C / gamma))^T
    unsigned short *Pb;   // [B][Hv][NC][2][C][C]  P hi, P lo
    // ... and for the bf16 backward sequential kernel
    unsigned short *PTb;  // [B][Hv][NC][2][C][C]  P^T hi, P^T lo
    unsigned short *QTb;  // [B][Hk][NC][D][C]     Q^T (per key head; per-channel gates: (Q * exp(G))^T per value head)
    unsigned short *nWTb; // [B][Hv][NC][D][C]     -W^T
    // per-channel gates (gdn_chunk_vg.hip): the cumulative log decays and the decayed operands that replace the row
    // scalings of the scalar-gate kernels (KTb then holds (K * exp(G_C - G))^T)
    float *Gv;            // [B][Hv][NC][C][D]     G_rj log2(e), G_rj = sum_{u<=r} log d_uj within the chunk; row C-1: G_C
    unsigned short *QGb;  // [B][Hv][NC][C][D]     Q * exp(G), fragment order (the forward's A operand of Y)
    unsigned short *KDb;  // [B][Hv][NC][C][D]     K * exp(G_C - G), fragment order (ck_bwd_seq's A operand of dDelta)
    // per-channel decays (not log decays): what ck_bwd_local_vg leaves for ck_vg_dg, VGD_FLOATS per chunk-head
    float *vgd;
};

// The vgd buffer of one chunk-head (fp32), by 16-token block R (rows 16R..16R+15, bt = 16R - 1, b2 = 16R + 15):
//   RHO [C][D]  exp(G_bt) rho0 + rho1: the pair terms through the chunk's entry state rho0 = q * dQg - beta k * Y2
//               and the row role through the token before the row's block rho1, before their decay factors
//   SIG [C][D]  exp(G_C - G_b2) sig0 + sig1: through the exit state sig0 = k * dKd and the column role through
//               the block's last token sig1
//   B0, B0P [4][D]  the block sums sum_{r in R} exp(G_r - G_bt) rho0_r and sum_{s in R} exp(G_b2 - G_s) sig0_s
//   dP, dA [C][C]   the pair cotangents (only the four diagonal blocks and the blocks (2, 0), (3, 0), (3, 1))
//   HD [D]      <dh', h> per state row
// The columns of RHO, SIG, B0 and B0P are in the permuted order of ck_bwd_local_vg's lanes: channel j at column
// (j & ~63) + 4 (j & 15) + ((j >> 4) & 3), so that each lane's four channels are one 16-byte piece.
constexpr int VGD_RHO = 0, VGD_SIG = VGD_RHO + C * D, VGD_B0 = VGD_SIG + C * D, VGD_B0P = VGD_B0 + 4 * D;
constexpr int VGD_DP = VGD_B0P + 4 * D, VGD_DA = VGD_DP + C * C, VGD_HD = VGD_DA + C * C, VGD_FLOATS = VGD_HD + D;

struct Args {
    const void *q, *k, *v;
    const float *g, *beta, *state0;
    const void *dy;
    const float *dstate_T;
    void *y, *dq, *dk, *dv;
    float *state_T, *dg, *dbeta, *dstate0;
    Bufs w;
    // A launch covers T tokens (NC chunks) of every sequence, starting at the token the input / output pointers
    // are offset to; Ts is the token stride of a sequence in those tensors (the full sequence length).  The
    // chunk buffers above are indexed by the launch's own chunks.
    int B, T, Ts, Hk, Hv, NC, in_dt, out_dt, dy_dt, grad_dt, gate;
    // Windows of wc chunks (0: none).  snap holds fp32 states [B][Hv][D][D] at the window boundaries, snapshot k
    // being the state entering window k + 1 of the sequence; win0 is the sequence window the launch starts at.
    //   forward (recompute = 0): the sequential forward writes snapshot win0 + c / wc - 1 on entering local
    //     chunk c > 0 with c % wc == 0;
    //   recompute = 1: the sequential forward runs grid.z = B * (windows in the launch), every window from its
    //     entry state (state0 for sequence window 0, else its snapshot), writing only H and Delta.
    float *snap;
    int wc, win0, recompute;
    int fwd_only;  // forward-only: ck_prep writes only the tiles the sequential forward reads
};

__device__ __forceinline__ size_t chunk_index(const Args &a, int b, int hv, int c) {
    return ((size_t)b * a.Hv + hv) * a.NC + c;
}

// What a sequential forward launch writes.  FWD_TRAIN: y, the final state and the tiles the backward reads (H,
// Delta); FWD_ONLY: y, the final state and the window snapshots (when Args::snap is set); FWD_RECOMPUTE: the windows
// of the launch side by side, H and Delta only (Args::recompute).
enum FwdMode { FWD_TRAIN = 0, FWD_ONLY = 1, FWD_RECOMPUTE = 2 };

// Chunks [cb, ce) and entry state of a sequential forward workgroup whose grid.z index is z.
struct SeqRange {
    int b, cb, ce;
    const float *s0;
};
template <int MODE>
__device__ __forceinline__ SeqRange seq_range(const Args &a, int z) {
    SeqRange r{z, 0, a.NC, a.state0};
    if constexpr (MODE == FWD_RECOMPUTE) {
        const int w = z / a.B, gw = a.win0 + w;
        r.b = z - w * a.B;
        r.cb = w * a.wc;
        r.ce = min(a.NC, r.cb + a.wc);
        r.s0 = gw == 0 ? a.state0 : a.snap + (size_t)(gw - 1) * a.B * a.Hv * D * D;
    }
    return r;
}

// The state slice a sequential workgroup holds in accumulators (rows j = 16 w + 4 lg + e, value columns
// i = i0 + 16 t + li) stored as S [head][i][j] fp32.
template <int NTN>
__device__ __forceinline__ void store_state_acc(float *dst, const f4 (&h)[NTN], size_t head, int i0, int w, int lg,
                                                int li) {
#pragma unroll
    for (int t = 0; t < NTN; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) dst[(head * D + i0 + 16 * t + li) * D + 16 * w + 4 * lg + e] = h[t][e];
}

// FWD_ONLY with windows: the snapshot taken on entering local chunk c, or NULL.
template <int MODE>
__device__ __forceinline__ float *snap_at(const Args &a, int c) {
    if (MODE != FWD_ONLY || !a.snap || a.wc <= 0 || c == 0 || c % a.wc) return nullptr;
    return a.snap + (size_t)(a.win0 + c / a.wc - 1) * a.B * a.Hv * D * D;
}

// Workgroups are dispatched to the 8 XCDs round-robin by linear id, and each XCD has its own L2.  The D / VS
// workgroups of one head in the sequential kernels read the same chunk tiles, so their linear id L is remapped to
// L' = (L mod 8) (N / 8) + L / 8 (N workgroups), which puts consecutive L' (the slices of one head) on one XCD,
// next to each other in its dispatch order.  The identity when N / 8 is not a multiple of the slices per head.
struct SeqBlock {
    int slice, hv, b;
};
__device__ __forceinline__ SeqBlock seq_block() {
    const int S = gridDim.x, Hv = gridDim.y, N = S * Hv * gridDim.z;
    int L = blockIdx.x + S * (blockIdx.y + Hv * blockIdx.z);
    if (N % 8 == 0 && (N / 8) % S == 0) L = (L % 8) * (N / 8) + L / 8;
    return {L % S, (L / S) % Hv, L / (S * Hv)};
}

// acc += X(16x16) * Y(16x16) on v_mfma_f32_16x16x4_f32; X, Y in LDS with row strides ldx, ldy.  Accumulator element
// e of lane l is (row 4*(l/16) + e, column l%16).
__device__ __forceinline__ void blk16_mma(f4 &acc, const float *X, int ldx, const float *Y, int ldy) {
    const int l = threadIdx.x & 63, li = l & 15, lg = l >> 4;
#pragma unroll
    for (int k0 = 0; k0 < 16; k0 += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(X[li * ldx + k0 + lg], Y[(k0 + lg) * ldy + li], acc, 0, 0, 0);
}

// (I + A)^-1 of a unit lower-triangular 64x64 matrix, A strictly lower in sA, in fp32.  Diagonal 16x16 blocks by
// column-parallel forward substitution; then the off-diagonal blocks by distance d = i - j on fp32 MFMA, one wave
// per block: T_ij = -T_ii sum_{u=j}^{i-1} A_iu T_uj (the inner sum goes through a wave-private 16x16 scratch to
// become an operand).  scratch holds 3 * 256 floats.  Ends with a barrier.
template <int NTH>
__device__ __forceinline__ void unit_lower_inverse(const float *sA, float *sT, float *scratch) {
    static_assert(NTH >= 3 * 64, "one wave per off-diagonal block of a round");
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, li = l & 15, lg = l >> 4;
    for (int i = tid; i < C * C; i += NTH) {
        const int r = i / C, s = i - r * C;
        if ((s >> 4) > (r >> 4)) sT[r * LDC + s] = 0.f;
    }
    if (tid < 64) {
        const int base = (tid >> 4) * 16, cc = tid & 15;
        // right-looking substitution: once x_u is final it updates every later row, so the dependency chain is
        // 16 multiply-adds long instead of 120 (each x_r still receives its terms in the order u = 0, 1, ...)
        float col[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) col[r] = (r == cc) ? 1.f : 0.f;
#pragma unroll
        for (int u = 0; u < 16; ++u)
#pragma unroll
            for (int r = u + 1; r < 16; ++r) col[r] = fmaf(-sA[(base + r) * LDC + base + u], col[u], col[r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) sT[(base + r) * LDC + base + cc] = col[r];
    }
    __syncthreads();
    for (int d = 1; d < 4; ++d) {
        if (w < 4 - d) {
            const int bj = w, bi = w + d;
            f4 x = zero4();
            for (int u = bj; u < bi; ++u) blk16_mma(x, sA + 16 * bi * LDC + 16 * u, LDC, sT + 16 * u * LDC + 16 * bj, LDC);
            float *sc = scratch + 256 * w;
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[(4 * lg + e) * 16 + li] = x[e];
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the wave's scratch writes before its reads
            f4 y = zero4();
            blk16_mma(y, sT + 16 * bi * LDC + 16 * bi, LDC, sc, 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) sT[(16 * bi + 4 * lg + e) * LDC + 16 * bj + li] = -y[e];
        }
        __syncthreads();
    }
}

// Threads per workgroup: ck_prep, the sequential kernels and ck_bwd_local all run 8 waves.
constexpr int NTP = 512;  // ck_prep: 8 waves
constexpr int NTS = 512;  // sequential kernels: 8 waves
constexpr int NTB = 512;  // ck_bwd_local: 8 waves; waves w and w+4 share the 16-row strip w%4 (column halves)

// Sum over the wave, the same in every lane: DPP row sums, then the four row totals read as scalars.
__device__ __forceinline__ float wave_sum(float x) {
    x = row16_allreduce(x);
    const auto lane = [](float v, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i)); };
    return (lane(x, 0) + lane(x, 16)) + (lane(x, 32) + lane(x, 48));
}

// ---------------------------------------------------------------------------------------------- bf16 tiles
//
// Operand tiles of v_mfma_f32_16x16x32_bf16 kept in LDS as bf16 with the reduction index k contiguous:
// element (m, k) at t[m * ld + k], ld = K + 8.  A lane's fragment (8 consecutive k of row m0 + l%16, starting
// at k0 + 8*(l/16)) is one 16-byte LDS read; the 16-byte row pad puts the 16 rows of a read in distinct bank
// groups.  A computed fp32 operand whose rounding reaches the outputs is kept as two tiles hi = bf16(x) and
// lo = bf16(x - hi), converted once when the tile is staged instead of at every use.
typedef unsigned short bfr;  // raw bf16 bits
constexpr int LA = D + 8;    // row stride of [*][128] tiles
constexpr int LB = C + 8;    // row stride of [*][64] tiles

__device__ __forceinline__ uint32_t bfbits(float x) { return __builtin_bit_cast(unsigned short, (__bf16)x); }
__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ uint32_t pk(float a, float b) { return bfbits(a) | (bfbits(b) << 16); }
// hi / lo halves of a pair
__device__ __forceinline__ void pk2(float a, float b, uint32_t &h, uint32_t &lo) {
    const uint32_t ha = bfbits(a), hb = bfbits(b);
    h = ha | (hb << 16);
    lo = bfbits(a - bf2f(ha)) | (bfbits(b - bf2f(hb)) << 16);
}

// Fragment order of the bf16 A-operand tiles that ck_prep writes for the sequential kernels (and the P tile
// ck_bwd_local reads): element (m, k) of an [M][K] tile sits at frag_off<K>(m, k), so that the 16-byte fragment lane
// l of a wave loads for rows m0..m0+15 and k0..k0+31 (m0 % 16 = k0 % 32 = 0) is at frag_off<K>(m0, k0) + 8 l and one
// load instruction of the wave reads 1 KiB contiguous (a row-major tile gives 16 rows x 64 bytes per instruction).
template <int K>
__device__ __forceinline__ int frag_off(int m, int k) {
    return (((m >> 4) * (K / 32) + (k >> 5)) * 64 + (m & 15) + 16 * ((k & 31) >> 3)) * 8 + (k & 7);
}
constexpr int FRAG_BLOCK = 64 * 8;  // elements of one wave's 16 x 32 fragment block
// Accumulator order of the fp32 U tile [C][D] (bf16 set): the four rows m0 + 4 (l / 16) .. +3 of column n0 + l % 16
// that lane l of a 16 x 16 MFMA accumulator tile holds are 16 contiguous bytes at acc_off(m0 + 4 (l / 16), n0 + l % 16)
// (m0, n0 multiples of 16), one wave's tile 1 KiB.
__device__ __forceinline__ int acc_off(int m, int n) {
    return (((m >> 4) * (D / 16) + (n >> 4)) * 64 + (n & 15) + 16 * ((m & 15) >> 2)) * 4 + (m & 3);
}

__device__ __forceinline__ bf8 frag(const bfr *t, int ld, int m0, int k0, int l = threadIdx.x & 63) {
    return *reinterpret_cast<const bf8 *>(t + (m0 + (l & 15)) * ld + k0 + 8 * (l >> 4));
}

// acc[t] += A(16 x K, rows m0.. of tile a) * B_t, B_t(k, n) = b[(n0 + 16 t + n) * ldb + k].  SA / SB add the lo
// parts of a split operand.
template <int K, int NTL, bool SA = false, bool SB = false>
__device__ __forceinline__ void mmab(f4 (&acc)[NTL], const bfr *ah, const bfr *al, int lda, int m0, const bfr *bh,
                                     const bfr *bl, int ldb, int n0, int l = threadIdx.x & 63) {
#pragma unroll 2
    for (int k0 = 0; k0 < K; k0 += 32) {
        // every fragment of the k-step is read before its first product, so the LDS reads overlap
        const bf8 x = frag(ah, lda, m0, k0, l);
        bf8 x2, y[NTL], y2[SB ? NTL : 1];
        if constexpr (SA) x2 = frag(al, lda, m0, k0, l);
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
            y[t] = frag(bh, ldb, n0 + 16 * t, k0, l);
            if constexpr (SB) y2[t] = frag(bl, ldb, n0 + 16 * t, k0, l);
        }
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y[t], acc[t], 0, 0, 0);
            if constexpr (SA) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x2, y[t], acc[t], 0, 0, 0);
            if constexpr (SB) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y2[t], acc[t], 0, 0, 0);
        }
    }
}

// Global [ROWS][COLS] (row stride `stride` elements, rows >= n read as zero; fp32 when F32 else bf16) ->
// LDS tile dst[r][c] (row stride ldd).  All of a thread's loads are issued before its LDS stores.
template <int ROWS, int COLS, int NTH, bool F32, bool SPLIT>
__device__ __forceinline__ void stage_N(bfr *hi, bfr *lo, int ldd, const void *src, size_t stride, int n) {
    constexpr int CPR = COLS / 8, NCH = ROWS * CPR, PER = (NCH + NTH - 1) / NTH;
    const int tid = threadIdx.x;
    uint4 raw[F32 ? 2 * PER : PER];
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int ch = tid + p * NTH, r = ch / CPR, c = (ch - r * CPR) * 8;
        const bool ok = ch < NCH && r < n;
        if constexpr (F32) {
            const float *s = static_cast<const float *>(src) + r * stride + c;
            raw[2 * p] = ok ? *reinterpret_cast<const uint4 *>(s) : make_uint4(0, 0, 0, 0);
            raw[2 * p + 1] = ok ? *reinterpret_cast<const uint4 *>(s + 4) : make_uint4(0, 0, 0, 0);
        } else {
            raw[p] = ok ? *reinterpret_cast<const uint4 *>(static_cast<const bfr *>(src) + r * stride + c)
                        : make_uint4(0, 0, 0, 0);
        }
    }
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int ch = tid + p * NTH, r = ch / CPR, c = (ch - r * CPR) * 8;
        if (ch >= NCH) break;
        if constexpr (F32) {
            const uint4 a = raw[2 * p], b = raw[2 * p + 1];
            uint4 h, l;
            pk2(__uint_as_float(a.x), __uint_as_float(a.y), h.x, l.x);
            pk2(__uint_as_float(a.z), __uint_as_float(a.w), h.y, l.y);
            pk2(__uint_as_float(b.x), __uint_as_float(b.y), h.z, l.z);
            pk2(__uint_as_float(b.z), __uint_as_float(b.w), h.w, l.w);
            *reinterpret_cast<uint4 *>(hi + r * ldd + c) = h;
            if constexpr (SPLIT) *reinterpret_cast<uint4 *>(lo + r * ldd + c) = l;
        } else {
            *reinterpret_cast<uint4 *>(hi + r * ldd + c) = raw[p];
        }
    }
}

// Global [ROWS][COLS] -> transposed LDS tile dst[c][r] (row stride ldd).  A thread moves an 8-row x 4-column
// block: 8 row loads, then 4 stores of 8 consecutive r.
template <int ROWS, int COLS, int NTH, bool F32, bool SPLIT>
__device__ __forceinline__ void stage_T(bfr *hi, bfr *lo, int ldd, const void *src, size_t stride, int n) {
    constexpr int CB = COLS / 4, NB = (ROWS / 8) * CB, PER = (NB + NTH - 1) / NTH;
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int blk = tid + p * NTH;
        if (blk >= NB) break;
        const int rb = blk / CB, c0 = (blk - rb * CB) * 4;
        float v[8][4];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const int r = rb * 8 + rr;
            if constexpr (F32) {
                const float4 x = r < n ? *reinterpret_cast<const float4 *>(static_cast<const float *>(src) + r * stride + c0)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
                v[rr][0] = x.x; v[rr][1] = x.y; v[rr][2] = x.z; v[rr][3] = x.w;
            } else {
                const uint2 x = r < n ? *reinterpret_cast<const uint2 *>(static_cast<const bfr *>(src) + r * stride + c0)
                                      : make_uint2(0, 0);
                v[rr][0] = bf2f(x.x & 0xffffu); v[rr][1] = bf2f(x.x >> 16);
                v[rr][2] = bf2f(x.y & 0xffffu); v[rr][3] = bf2f(x.y >> 16);
            }
        }
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            uint4 h, l;
            pk2(v[0][cc], v[1][cc], h.x, l.x);
            pk2(v[2][cc], v[3][cc], h.y, l.y);
            pk2(v[4][cc], v[5][cc], h.z, l.z);
            pk2(v[6][cc], v[7][cc], h.w, l.w);
            *reinterpret_cast<uint4 *>(hi + (c0 + cc) * ldd + rb * 8) = h;
            if constexpr (SPLIT) *reinterpret_cast<uint4 *>(lo + (c0 + cc) * ldd + rb * 8) = l;
        }
    }
}

// Global [ROWS][COLS] -> natural tile N[r][c] (ldn, hi only) and transposed tile Tt[c][r] (ldt) from one load
// of each element (8-row x 4-column blocks per thread).
template <int ROWS, int COLS, int NTH, bool F32, bool SPLIT_T>
__device__ __forceinline__ void stage_NT(bfr *nh, int ldn, bfr *th, bfr *tl, int ldt, const void *src, size_t stride,
                                         int n) {
    constexpr int CB = COLS / 4, NB = (ROWS / 8) * CB, PER = (NB + NTH - 1) / NTH;
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int blk = tid + p * NTH;
        if (blk >= NB) break;
        const int rb = blk / CB, c0 = (blk - rb * CB) * 4;
        float v[8][4];
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const int r = rb * 8 + rr;
            if constexpr (F32) {
                const float4 x = r < n ? *reinterpret_cast<const float4 *>(static_cast<const float *>(src) + r * stride + c0)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
                v[rr][0] = x.x; v[rr][1] = x.y; v[rr][2] = x.z; v[rr][3] = x.w;
            } else {
                const uint2 x = r < n ? *reinterpret_cast<const uint2 *>(static_cast<const bfr *>(src) + r * stride + c0)
                                      : make_uint2(0, 0);
                v[rr][0] = bf2f(x.x & 0xffffu); v[rr][1] = bf2f(x.x >> 16);
                v[rr][2] = bf2f(x.y & 0xffffu); v[rr][3] = bf2f(x.y >> 16);
            }
        }
#pragma unroll
        for (int rr = 0; rr < 8; ++rr)
            *reinterpret_cast<uint2 *>(nh + (rb * 8 + rr) * ldn + c0) = make_uint2(pk(v[rr][0], v[rr][1]), pk(v[rr][2], v[rr][3]));
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            uint4 h, l;
            pk2(v[0][cc], v[1][cc], h.x, l.x);
            pk2(v[2][cc], v[3][cc], h.y, l.y);
            pk2(v[4][cc], v[5][cc], h.z, l.z);
            pk2(v[6][cc], v[7][cc], h.w, l.w);
            *reinterpret_cast<uint4 *>(th + (c0 + cc) * ldt + rb * 8) = h;
            if constexpr (SPLIT_T) *reinterpret_cast<uint4 *>(tl + (c0 + cc) * ldt + rb * 8) = l;
        }
    }
}

// The bf16 chunk states h and dh' ([D][D] as [j][i]) -> LDS tiles, returning this thread's part of the inner
// product <dh', h> (fp32 sums of the bf16 products).
template <int NTH>
__device__ __forceinline__ float stage_states(bfr *hh, bfr *dhh, const bfr *H, const bfr *dH) {
    constexpr int CPR = D / 8, NCH = D * CPR, PER = NCH / NTH;
    static_assert(PER * NTH == NCH, "even split");
    const int tid = threadIdx.x;
    uint4 hv[PER], dv[PER];
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int ch = tid + p * NTH;
        hv[p] = reinterpret_cast<const uint4 *>(H)[ch];
        dv[p] = reinterpret_cast<const uint4 *>(dH)[ch];
    }
    float dot = 0.f;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
        const int ch = tid + p * NTH, r = ch / CPR, c = (ch - r * CPR) * 8;
        *reinterpret_cast<uint4 *>(hh + r * LA + c) = hv[p];
        *reinterpret_cast<uint4 *>(dhh + r * LA + c) = dv[p];
        const uint32_t hw[4] = {hv[p].x, hv[p].y, hv[p].z, hv[p].w}, dw[4] = {dv[p].x, dv[p].y, dv[p].z, dv[p].w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
            dot += bf2f(hw[q] & 0xffffu) * bf2f(dw[q] & 0xffffu) + bf2f(hw[q] >> 16) * bf2f(dw[q] >> 16);
    }
    return dot;
}

// An 8-row x 4-column block of a global bf16 [ROWS][COLS] tile (rows >= n read as zero), kept as the raw loads
// so that a phase can issue all of its loads before the first LDS store.
struct Blk84 {
    uint2 raw[8];
    int rb, c0;
    __device__ __forceinline__ void load(const bfr *src, size_t stride, int blk, int cols, int n) {
        rb = blk / (cols / 4);
        c0 = (blk - rb * (cols / 4)) * 4;
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const int r = rb * 8 + rr;
            raw[rr] = r < n ? *reinterpret_cast<const uint2 *>(src + r * stride + c0) : make_uint2(0u, 0u);
        }
    }
    __device__ __forceinline__ uint32_t e16(int rr, int cc) const {
        const uint32_t w = cc < 2 ? raw[rr].x : raw[rr].y;
        return cc & 1 ? w >> 16 : w & 0xffffu;
    }
    // dst[c][r]: four stores of 8 consecutive rows
    __device__ __forceinline__ void store_T(bfr *dst, int ldt) const {
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
            *reinterpret_cast<uint4 *>(dst + (c0 + cc) * ldt + rb * 8) =
                make_uint4(e16(0, cc) | (e16(1, cc) << 16), e16(2, cc) | (e16(3, cc) << 16),
                           e16(4, cc) | (e16(5, cc) << 16), e16(6, cc) | (e16(7, cc) << 16));
    }
    // dst[r][c]: eight stores of 4 consecutive columns
    __device__ __forceinline__ void store_N(bfr *nh, int ldn) const {
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) *reinterpret_cast<uint2 *>(nh + (rb * 8 + rr) * ldn + c0) = raw[rr];
    }
};

// MFMA accumulator tile X (rows m0 + 4(l/16) + e, column n0 + l%16) -> LDS, transposed (dst[n][m]: four
// consecutive bf16 per lane) or natural (dst[m][n]).
template <bool SPLIT>
__device__ __forceinline__ void acc_T(const f4 &x, bfr *hi, bfr *lo, int ld, int m0, int n0, int l = threadIdx.x & 63) {
    const int o = (n0 + (l & 15)) * ld + m0 + 4 * (l >> 4);
    uint2 h, lw;
    pk2(x[0], x[1], h.x, lw.x);
    pk2(x[2], x[3], h.y, lw.y);
    *reinterpret_cast<uint2 *>(hi + o) = h;
    if constexpr (SPLIT) *reinterpret_cast<uint2 *>(lo + o) = lw;
}
template <bool SPLIT>
__device__ __forceinline__ void acc_N(const f4 &x, bfr *hi, bfr *lo, int ld, int m0, int n0, int l = threadIdx.x & 63) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int o = (m0 + 4 * (l >> 4) + e) * ld + n0 + (l & 15);
        const uint32_t h = bfbits(x[e]);
        hi[o] = (bfr)h;
        if constexpr (SPLIT) lo[o] = (bfr)bfbits(x[e] - bf2f(h));
    }
}

// ---------------------------------------------------------------------------------------------- register fragments
//
// MFMA A operands loaded as fragments straight from global memory into registers.
__device__ __forceinline__ bf8 ld_frag(const bfr *p) { return *reinterpret_cast<const bf8 *>(p); }
__device__ __forceinline__ bf8 zero_frag() { return __builtin_bit_cast(bf8, make_uint4(0u, 0u, 0u, 0u)); }

// acc[t] += A * B_t with the A fragments of the K/32 k-steps in registers (ah[k], al[k] for the lo part).
template <int K, int NTL, bool SA = false, bool SB = false>
__device__ __forceinline__ void mmar(f4 (&acc)[NTL], const bf8 *ah, const bf8 *al, const bfr *bh, const bfr *bl,
                                     int ldb, int n0) {
#pragma unroll
    for (int k = 0; k < K / 32; ++k) {
        // the k-step's LDS fragments are all read before its first product: one LDS round trip per k-step
        bf8 y[NTL], y2[SB ? NTL : 1];
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
            y[t] = frag(bh, ldb, n0 + 16 * t, 32 * k);
            if constexpr (SB) y2[t] = frag(bl, ldb, n0 + 16 * t, 32 * k);
        }
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[k], y[t], acc[t], 0, 0, 0);
            if constexpr (SA) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[k], y[t], acc[t], 0, 0, 0);
            if constexpr (SB) acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[k], y2[t], acc[t], 0, 0, 0);
        }
    }
}

// Per-channel-gate stages of the bf16 set (gdn_chunk_vg.hip).
void launch_vg_prep(const Args &a, hipStream_t st);
void launch_vg_local(const Args &a, hipStream_t st);
void launch_vg_dg(const Args &a, hipStream_t st);  // per-channel decays only: d/d(decay) after launch_vg_local

}  // namespace ck
}  // namespace gdn
