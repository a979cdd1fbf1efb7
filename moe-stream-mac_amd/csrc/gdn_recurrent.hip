// Token-sequential ("recurrent") form of the Gated DeltaNet forward and VJP for gfx950.
//
// Work split.  The rows of the [Dv][Dk] state are independent in the forward (engine/include/gdn.h:36), so a
// workgroup owns one (batch, value head, block of 16 value rows).  Each row lives in the VGPRs of one DPP row
// of 16 lanes, E = Dk/16 key channels per lane; row dot products (S k, S q, dS~ k) are 4-step DPP all-reduces
// with no LDS traffic and no barriers.  Per-token inputs are staged through LDS in tiles.
//
// Backward.  Reverse-time adjoint of tools/gdn_vjp.py:8-21 (_chunk_vjp :273-320).  The states inside a chunk
// are never stored: for each chunk the workgroup reloads the chunk-start snapshot written by the forward,
// replays the chunk once to write sub-chunk starts (every CS tokens) to a small workspace, then for each
// sub-chunk in reverse replays CS steps keeping S_{t-1} of its rows in VGPRs (fully unrolled), and walks them
// backward.  Backward workgroups hold 16 or 32 rows (4 or 8 waves; rec_bwd_rows).  Cross-row sums (dq, dk, dg,
// dbeta) are reduced in-wave (lane swaps), across the waves in LDS, and across row blocks and the GQA head group by
// a second, deterministic kernel — no atomics.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {

constexpr int ROWS = 16;      // value rows per workgroup (16 DPP rows of 16 lanes)
constexpr int THREADS = 256;  // 4 wave64
constexpr int FWD_TT = 16;    // tokens per LDS tile in the forward
constexpr int BWD_CS = 8;     // tokens per register-resident sub-chunk in the backward

template <int E, bool VEC, int TT, int R>
struct StageBuf {
    static constexpr int DKP = 16 * E;
    float k[TT][DKP];
    float q[TT][DKP];
    float g[TT][VEC ? DKP : 1];
    float v[TT][R];
    float dy[TT][R];
    float beta[TT];
    float m[TT];
};

// One thread's share of a stage of TT tokens, in registers: stage_fetch issues every load of the stage at once,
// stage_store moves them to LDS.  The loads take clamped indices (a token past T reads token T - 1, a channel or
// row past Dk / Dv the last one) and sit under no branch, and the dtypes are template parameters: loads under a
// branch or a dtype switch made the compiler wait for each one where the branches joined, so a stage's loads came
// in one after another.  stage_store zeroes what lies past the tokens, channels and rows (decay 1), so padded
// lanes carry exact zeros through every step.
// NT threads stage the tokens of a workgroup of R value rows.
template <int E, bool VEC, int TT, bool WITH_DY, int NT, int R>
struct TokRegs {
    static constexpr int DKP = 16 * E;
    static constexpr int NKQ = (TT * DKP + NT - 1) / NT;
    static constexpr int NV = (TT * R + NT - 1) / NT;
    float k[NKQ], q[NKQ], g[VEC ? NKQ : 1], v[NV], dy[WITH_DY ? NV : 1];
    float bt, gt, mt;
};

template <int E, bool VEC, int TT, bool WITH_DY, int DT, int DYT, int NT, int R>
__device__ __forceinline__ void stage_fetch(TokRegs<E, VEC, TT, WITH_DY, NT, R> &r, const void *q, const void *k,
                                            const void *v, const float *g, const float *beta, const uint8_t *mask,
                                            const void *dy, int b, int hv, int hk, int rb, int t0, int T, int Hk,
                                            int Hv, int Dk, int Dv, int in_dt, int dy_dt) {
    using TR = TokRegs<E, VEC, TT, WITH_DY, NT, R>;
    const int tid = threadIdx.x;
    const int xdt = DT >= 0 ? DT : in_dt, ydt = DYT >= 0 ? DYT : dy_dt;  // DT < 0: read from the arguments
#pragma unroll
    for (int p = 0; p < TR::NKQ; ++p) {
        const int i = tid + p * NT, tt = i / TR::DKP, j = i - tt * TR::DKP;
        const int t = min(t0 + tt, T - 1), jc = min(j, Dk - 1);
        const size_t idx = (((size_t)b * T + t) * Hk + hk) * Dk + jc;
        r.k[p] = load_as_f32(k, idx, xdt);
        r.q[p] = load_as_f32(q, idx, xdt);
        if constexpr (VEC) r.g[p] = g[(((size_t)b * T + t) * Hv + hv) * Dk + jc];
    }
#pragma unroll
    for (int p = 0; p < TR::NV; ++p) {
        const int i = tid + p * NT, tt = i / R, rr = rb * R + (i - tt * R);
        const size_t idx = (((size_t)b * T + min(t0 + tt, T - 1)) * Hv + hv) * Dv + min(rr, Dv - 1);
        r.v[p] = load_as_f32(v, idx, xdt);
        if constexpr (WITH_DY) r.dy[p] = load_as_f32(dy, idx, ydt);
    }
    const int t = min(t0 + tid % TT, T - 1);
    const size_t gi = ((size_t)b * T + t) * Hv + hv;
    r.bt = beta[gi];
    if constexpr (!VEC) r.gt = g[gi];
    // without a mask, a byte of beta is read in its place (and ignored): no branch around the load
    const uint8_t *mp = mask ? mask + (size_t)b * T + t : reinterpret_cast<const uint8_t *>(beta + gi);
    r.mt = *mp ? 1.f : 0.f;
}

template <int E, bool VEC, int TT, bool WITH_DY, int NT, int R>
__device__ __forceinline__ void stage_store(StageBuf<E, VEC, TT, R> &sb,
                                            const TokRegs<E, VEC, TT, WITH_DY, NT, R> &r, bool masked, int n, int Dk,
                                            int Dv, int rb, int gate) {
    using TR = TokRegs<E, VEC, TT, WITH_DY, NT, R>;
    const int tid = threadIdx.x;
#pragma unroll
    for (int p = 0; p < TR::NKQ; ++p) {
        const int i = tid + p * NT, tt = i / TR::DKP, j = i - tt * TR::DKP;
        if (i < TT * TR::DKP) {
            const bool ok = tt < n && j < Dk;
            sb.k[tt][j] = ok ? r.k[p] : 0.f;
            sb.q[tt][j] = ok ? r.q[p] : 0.f;
            if constexpr (VEC) sb.g[tt][j] = ok ? (gate == GATE_LOG_VEC ? expf(r.g[p]) : r.g[p]) : 1.f;
        }
    }
#pragma unroll
    for (int p = 0; p < TR::NV; ++p) {
        const int i = tid + p * NT, tt = i / R, rl = i - tt * R;
        if (i < TT * R) {
            const bool ok = tt < n && rb * R + rl < Dv;
            sb.v[tt][rl] = ok ? r.v[p] : 0.f;
            if constexpr (WITH_DY) sb.dy[tt][rl] = ok ? r.dy[p] : 0.f;
        }
    }
    if (tid < TT) {
        const bool ok = tid < n;
        sb.beta[tid] = ok ? r.bt : 0.f;
        if constexpr (!VEC) sb.g[tid][0] = ok ? (gate == GATE_LOG ? expf(r.gt) : r.gt) : 1.f;
        sb.m[tid] = ok && masked ? r.mt : 1.f;
    }
}

template <int E>
__device__ __forceinline__ void lds_vec(float (&dst)[E], const float *src) {
    if constexpr (E % 4 == 0) {
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            const float4 x = *reinterpret_cast<const float4 *>(src + e);
            dst[e] = x.x; dst[e + 1] = x.y; dst[e + 2] = x.z; dst[e + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) dst[e] = src[e];
    }
}

// One forward step of one state row held as E channels per lane.  Returns the residual r = v - A k and
// leaves the candidate S~ in cand.
template <int E, bool VEC, int TT, int R>
__device__ __forceinline__ float row_step(const StageBuf<E, VEC, TT, R> &sb, int tt, int grp, int c,
                                          const float (&S)[E], float (&cand)[E], float (&kk)[E],
                                          float &delta) {
    float dec[E];
    lds_vec<E>(kk, &sb.k[tt][c * E]);
    if (VEC) {
        lds_vec<E>(dec, &sb.g[tt][c * E]);
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) dec[e] = sb.g[tt][0];
    }
    float A[E];
    float kv = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        A[e] = S[e] * dec[e];
        kv = fmaf(A[e], kk[e], kv);
    }
    kv = row16_allreduce(kv);
    const float r = sb.v[tt][grp] - kv;
    delta = r * sb.beta[tt];
#pragma unroll
    for (int e = 0; e < E; ++e) cand[e] = fmaf(delta, kk[e], A[e]);
    return r;
}

// ---------------------------------------------------------------------------------------------------- forward

// MASKED: a mask is given (without one every token keeps its candidate state and the selects compile away).
template <int E, bool VEC, int DT, bool MASKED>
__global__ __launch_bounds__(THREADS) void rec_fwd_kernel(RecFwdArgs a) {
    __shared__ __align__(16) StageBuf<E, VEC, FWD_TT, ROWS> sb;
    __shared__ float s_y[FWD_TT][ROWS];

    const int rb = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, grp = tid >> 4, c = tid & 15;
    const int row = rb * ROWS + grp;
    const bool row_ok = row < a.Dv;
    const int hk = hv / (a.Hv / a.Hk);
    const int T = a.T, Dk = a.Dk, Dv = a.Dv;
    const size_t state_elems = (size_t)a.B * a.Hv * Dv * Dk;
    const size_t row_off = (((size_t)b * a.Hv + hv) * Dv + row) * Dk;

    float S[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int j = c * E + e;
        S[e] = (a.state0 && row_ok && j < Dk) ? a.state0[row_off + j] : 0.f;
    }
    int until_snap = a.chunk;  // tokens left before the next chunk boundary
    // the next stage's tokens are loaded into registers while this one computes
    TokRegs<E, VEC, FWD_TT, false, THREADS, ROWS> tr;
    auto fetch = [&](int t0) {
        stage_fetch<E, VEC, FWD_TT, false, DT, DT, THREADS, ROWS>(tr, a.q, a.k, a.v, a.g, a.beta, a.mask, nullptr, b,
                                                                  hv, hk, rb, t0, T, a.Hk, a.Hv, Dk, Dv, a.in_dt, 0);
    };
    fetch(0);
    for (int t0 = 0; t0 < T; t0 += FWD_TT) {
        const int n = min(FWD_TT, T - t0);
        __syncthreads();
        stage_store<E, VEC, FWD_TT, false, THREADS, ROWS>(sb, tr, a.mask != nullptr, n, Dk, Dv, rb, a.gate);
        __syncthreads();
        fetch(t0 + FWD_TT);
        auto token = [&](const int tt) {
            float cand[E], kk[E], qq[E], delta;
            row_step<E, VEC, FWD_TT, ROWS>(sb, tt, grp, c, S, cand, kk, delta);
            lds_vec<E>(qq, &sb.q[tt][c * E]);
            float y = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) y = fmaf(cand[e], qq[e], y);
            y = row16_allreduce(y);
            const bool keep = !MASKED || sb.m[tt] != 0.f;  // a select, not a branch: no register shuffles around it
#pragma unroll
            for (int e = 0; e < E; ++e) S[e] = keep ? cand[e] : S[e];
            if (c == 0) s_y[tt][grp] = y;
            if (--until_snap == 0) {
                until_snap = a.chunk;
                const int t = t0 + tt;
                if (a.snaps && t + 1 < T && row_ok) {
                    float *dst = a.snaps + (size_t)((t + 1) / a.chunk - 1) * state_elems + row_off;
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        const int j = c * E + e;
                        if (j < Dk) dst[j] = S[e];
                    }
                }
            }
        };
        // A full stage is unrolled, so each token's LDS reads are issued during the token before; a partial one
        // (the last, or a decode step's single token) steps only its n tokens.
        if (n == FWD_TT) {
#pragma unroll
            for (int tt = 0; tt < FWD_TT; ++tt) token(tt);
        } else {
            for (int tt = 0; tt < n; ++tt) token(tt);
        }
        __syncthreads();
        for (int i = tid; i < n * ROWS; i += THREADS) {
            const int tt = i / ROWS, r = i - tt * ROWS, rr = rb * ROWS + r;
            if (rr < Dv)
                store_from_f32(a.y, (((size_t)b * T + t0 + tt) * a.Hv + hv) * Dv + rr, s_y[tt][r], a.out_dt);
        }
    }
    if (a.state_T && row_ok) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int j = c * E + e;
            if (j < Dk) a.state_T[row_off + j] = S[e];
        }
    }
}

// ---------------------------------------------------------------------------------------------------- decode

// E consecutive elements from index i0 (16-byte aligned) as float: 16-byte loads when the dtype is fixed at compile
// time (8 bf16 or 4 fp32 per load), element loads otherwise.
template <int E, int DT>
__device__ __forceinline__ void load_span(float (&dst)[E], const void *p, size_t i0, int dt) {
    if constexpr (DT == DT_BF16 && E % 8 == 0) {
#pragma unroll
        for (int e = 0; e < E; e += 8) {
            const uint4 x = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + i0 + e);
            const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                dst[e + 2 * u] = __uint_as_float(w[u] << 16);
                dst[e + 2 * u + 1] = __uint_as_float(w[u] & 0xffff0000u);
            }
        }
    } else if constexpr (DT == DT_F32 && E % 4 == 0) {
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            const float4 x = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i0 + e);
            dst[e] = x.x; dst[e + 1] = x.y; dst[e + 2] = x.z; dst[e + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) dst[e] = load_as_f32(p, i0 + e, dt);
    }
}

// One token of B sequences (gdn_decode_step, engine/src/gdn.c:63-108): the forward step with every input read
// straight into registers, no LDS and no barrier, so the launch streams the state.  A lane loads its E channels of
// k and q (clamped, zero past Dk), its row's v, the head's beta and decay, and its E state elements; it computes in
// the forward kernel's order of operations (the same results) and writes the state back, which may be in place
// (a lane reads its elements before writing them).  Without state0 the state is zero: state_T is read in its place
// (in bounds, unused), so no load sits under a branch.
template <int E, bool VEC, int DT>
__global__ __launch_bounds__(THREADS) void rec_decode_kernel(RecFwdArgs a) {
    const int rb = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, grp = tid >> 4, c = tid & 15;
    const int Dk = a.Dk, Dv = a.Dv, row = rb * ROWS + grp, rowc = min(row, Dv - 1);
    const bool row_ok = row < Dv, has0 = a.state0 != nullptr;
    const int hk = hv / (a.Hv / a.Hk), xdt = DT >= 0 ? DT : a.in_dt;
    const size_t head = (size_t)b * a.Hv + hv, kq0 = ((size_t)b * a.Hk + hk) * Dk;
    const size_t row_off = (head * Dv + rowc) * Dk;
    const float *s_in = has0 ? a.state0 : a.state_T;
    // full rows of 16-byte pieces: E % 4 == 0, Dk = 16 E, both state rows aligned
    const uintptr_t align = reinterpret_cast<uintptr_t>(s_in) | reinterpret_cast<uintptr_t>(a.state_T) |
                            reinterpret_cast<uintptr_t>(a.k) | reinterpret_cast<uintptr_t>(a.q);
    const bool wide = E % 4 == 0 && Dk == 16 * E && (align & 15) == 0;
    float kk[E], qq[E], dec[E], S[E];
    const float vr = load_as_f32(a.v, head * Dv + rowc, xdt), bt = a.beta[head];
    const float gs = VEC ? 1.f : a.g[head];
    const float dsc = a.gate == GATE_LOG ? expf(gs) : gs;
    if (wide) {  // 16-byte pieces of the state row and of k and q (every channel valid)
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            const float4 x = *reinterpret_cast<const float4 *>(s_in + row_off + c * E + e);
            S[e] = x.x; S[e + 1] = x.y; S[e + 2] = x.z; S[e + 3] = x.w;
        }
        load_span<E, DT>(kk, a.k, kq0 + c * E, xdt);
        load_span<E, DT>(qq, a.q, kq0 + c * E, xdt);
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int jc = min(c * E + e, Dk - 1);
            S[e] = s_in[row_off + jc];
            kk[e] = load_as_f32(a.k, kq0 + jc, xdt);
            qq[e] = load_as_f32(a.q, kq0 + jc, xdt);
        }
    }
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int j = c * E + e, jc = min(j, Dk - 1);
        const bool ok = j < Dk;
        kk[e] = ok ? kk[e] : 0.f;
        qq[e] = ok ? qq[e] : 0.f;
        if constexpr (VEC) {
            const float gx = a.g[head * Dk + jc];
            dec[e] = ok ? (a.gate == GATE_LOG_VEC ? expf(gx) : gx) : 1.f;
        } else {
            dec[e] = dsc;
        }
        S[e] = has0 && ok && row_ok ? S[e] : 0.f;
    }
    float A[E], kv = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        A[e] = S[e] * dec[e];
        kv = fmaf(A[e], kk[e], kv);
    }
    kv = row16_allreduce(kv);
    const float delta = ((row_ok ? vr : 0.f) - kv) * bt;
    float y = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        S[e] = fmaf(delta, kk[e], A[e]);
        y = fmaf(S[e], qq[e], y);
    }
    y = row16_allreduce(y);
    if (row_ok) {
        if (wide) {
#pragma unroll
            for (int e = 0; e < E; e += 4)
                *reinterpret_cast<float4 *>(a.state_T + row_off + c * E + e) =
                    make_float4(S[e], S[e + 1], S[e + 2], S[e + 3]);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e)
                if (c * E + e < Dk) a.state_T[row_off + c * E + e] = S[e];
        }
        if (c == 0) store_from_f32(a.y, head * Dv + row, y, a.out_dt);
    }
}

// ---------------------------------------------------------------------------------------------------- backward

// NW waves per workgroup, 4 NW value rows (4 per wave).  MASKED as in the forward.
template <int E, bool VEC, int DT, int NW, bool MASKED>
__global__ __launch_bounds__(64 * NW) void rec_bwd_kernel(RecBwdArgs a) {
    constexpr int CS = BWD_CS;
    constexpr int DKP = 16 * E;
    constexpr int NQ = VEC ? 3 : 2;
    constexpr int NT = 64 * NW, R = 4 * NW;
    __shared__ __align__(16) StageBuf<E, VEC, CS, R> sb;
    __shared__ __align__(16) float s_red[CS][NW][NQ * DKP];  // per wave, sums over its 4 rows: dq | dk | (dg / channel)
    __shared__ float s_row[CS][R][3];                        // per row: dv, dbeta, dg (scalar gate)

    const int rb = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, grp = tid >> 4, c = tid & 15, wave = tid >> 6, gw = grp & 3;
    const int row = rb * R + grp;
    const bool row_ok = row < a.Dv;
    const int hk = hv / (a.Hv / a.Hk);
    const int T = a.T, Dk = a.Dk, Dv = a.Dv, B = a.B, Hv = a.Hv;
    const size_t state_elems = (size_t)B * Hv * Dv * Dk;
    const size_t row_off = (((size_t)b * Hv + hv) * Dv + row) * Dk;
    float *ws = a.ws_sub + ((((size_t)b * Hv + hv) * a.nrb + rb) * a.max_sub) * R * DKP + grp * DKP + c * E;
    // rows of whole 16-byte pieces in the partial-sum buffers
    const bool part_vec = (Dk & 3) == 0 && (reinterpret_cast<uintptr_t>(a.part_qk) & 15) == 0 &&
                          (!VEC || (reinterpret_cast<uintptr_t>(a.part_gv) & 15) == 0);

    float dS[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int j = c * E + e;
        dS[e] = (a.dstate_T && row_ok && j < Dk) ? a.dstate_T[row_off + j] : 0.f;
    }
    const int nch = (T + a.chunk - 1) / a.chunk;
    // Stages in order: per chunk (last first), the replay sub-chunks 0 .. nsub-2, then the sub-chunks nsub-1 .. 0
    // with dY.  Each stage's tokens are loaded into registers during the stage before.
    TokRegs<E, VEC, CS, true, NT, R> tr;
    auto fetch = [&](int t0) {
        stage_fetch<E, VEC, CS, true, DT, DT, NT, R>(tr, a.q, a.k, a.v, a.g, a.beta, a.mask, a.dy, b, hv, hk, rb, t0,
                                                     T, a.Hk, Hv, Dk, Dv, a.in_dt, a.dy_dt);
    };
    fetch((nch - 1) * a.chunk);
    for (int ci = nch - 1; ci >= 0; --ci) {
        const int cs = ci * a.chunk, ce = min(T, cs + a.chunk);
        const int nsub = (ce - cs + CS - 1) / CS;
        const int next_chunk_t0 = ci > 0 ? (ci - 1) * a.chunk : 0;  // the previous chunk's first stage
        const float *start = ci == 0 ? a.state0 : a.snaps + (size_t)(ci - 1) * state_elems;
        float S[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int j = c * E + e;
            S[e] = (start && row_ok && j < Dk) ? start[row_off + j] : 0.f;
        }
        // Replay the chunk once, recording the state at each sub-chunk start (1 .. nsub-1).
        for (int si = 0; si < nsub - 1; ++si) {
            __syncthreads();
            stage_store<E, VEC, CS, true, NT, R>(sb, tr, a.mask != nullptr, CS, Dk, Dv, rb, a.gate);
            __syncthreads();
            fetch(si + 1 < nsub - 1 ? cs + (si + 1) * CS : cs + (nsub - 1) * CS);
#pragma unroll
            for (int s = 0; s < CS; ++s) {
                float cand[E], kk[E], delta;
                row_step<E, VEC, CS, R>(sb, s, grp, c, S, cand, kk, delta);
                const bool keep = !MASKED || sb.m[s] != 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) S[e] = keep ? cand[e] : S[e];
            }
#pragma unroll
            for (int e = 0; e < E; ++e) ws[(size_t)si * R * DKP + e] = S[e];
        }
        // Sub-chunks in reverse.
        for (int si = nsub - 1; si >= 0; --si) {
            const int ss = cs + si * CS, n = min(CS, ce - ss);
            if (si == 0) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int j = c * E + e;
                    S[e] = (start && row_ok && j < Dk) ? start[row_off + j] : 0.f;
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) S[e] = ws[(size_t)(si - 1) * R * DKP + e];
            }
            __syncthreads();
            stage_store<E, VEC, CS, true, NT, R>(sb, tr, a.mask != nullptr, n, Dk, Dv, rb, a.gate);
            __syncthreads();
            fetch(si > 0 ? cs + (si - 1) * CS : next_chunk_t0);
            // All CS slots are stepped, also past n: stage_store gives those k = v = beta = 0, decay 1 and keep 1,
            // so they leave S and dS unchanged, and their dq / dk / dg sums are never written out.
            float hist[CS][E];
            float rh[CS];
#pragma unroll
            for (int s = 0; s < CS; ++s) {
                float cand[E], kk[E], delta;
#pragma unroll
                for (int e = 0; e < E; ++e) hist[s][e] = S[e];
                rh[s] = row_step<E, VEC, CS, R>(sb, s, grp, c, S, cand, kk, delta);
                const bool keep = !MASKED || sb.m[s] != 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) S[e] = keep ? cand[e] : S[e];
            }
#pragma unroll
            for (int s = CS - 1; s >= 0; --s) {
                float kk[E], qq[E], dec[E];
                lds_vec<E>(kk, &sb.k[s][c * E]);
                lds_vec<E>(qq, &sb.q[s][c * E]);
                if (VEC) {
                    lds_vec<E>(dec, &sb.g[s][c * E]);
                } else {
#pragma unroll
                    for (int e = 0; e < E; ++e) dec[e] = sb.g[s][0];
                }
                const float dyr = sb.dy[s][grp], bt = sb.beta[s], r = rh[s], delta = r * bt;
                const bool keep = !MASKED || sb.m[s] != 0.f;
                float dSc[E];
                float u = 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    dSc[e] = fmaf(dyr, qq[e], keep ? dS[e] : 0.f);
                    u = fmaf(dSc[e], kk[e], u);
                }
                u = row16_allreduce(u);
                const float ev = bt * u;
                float pq[E], pk[E], pg[E];
                float dgl = 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const float A = hist[s][e] * dec[e];
                    const float cand = fmaf(delta, kk[e], A);
                    pq[e] = dyr * cand;
                    pk[e] = fmaf(dSc[e], delta, -ev * A);
                    const float dA = fmaf(-ev, kk[e], dSc[e]);
                    if (VEC) pg[e] = dA * hist[s][e];
                    else dgl = fmaf(dA, hist[s][e], dgl);
                    dS[e] = fmaf(dA, dec[e], keep ? 0.f : dS[e]);
                }
                if (!VEC) dgl = row16_allreduce(dgl);
                if (c == 0) {
                    s_row[s][grp][0] = ev;
                    s_row[s][grp][1] = u * r;
                    s_row[s][grp][2] = dgl;
                }
                // Sum dq / dk over the 4 rows of this wave: halve the vector at each exchange so every
                // lane ends with E/2 fully reduced values (even rows dq, odd rows dk; then the lower half
                // of the wave the first E/2 channels, the upper half the rest).
                const int h = gw & 1, h2 = gw >> 1;
                float W[E];
#pragma unroll
                for (int e = 0; e < E; ++e) W[e] = pair_sum16(pq[e], pk[e]);
                if constexpr (E >= 2) {
                    constexpr int H = E / 2;
#pragma unroll
                    for (int e = 0; e < H; ++e)
                        s_red[s][wave][h * DKP + c * E + h2 * H + e] = pair_sum32(W[e], W[H + e]);
                } else {
                    const float x = W[0] + lane_xor32(W[0]);
                    if (h2 == 0) s_red[s][wave][h * DKP + c] = x;
                }
                if constexpr (VEC) {
                    // the same halving over one vector: lane (h, h2) ends with channels
                    // c E + h E/2 + h2 E/4 + i, i < E/4, summed over the 4 rows
                    if constexpr (E >= 4) {
                        constexpr int H = E / 2, Q = E / 4;
                        float P[H];
#pragma unroll
                        for (int i = 0; i < H; ++i) P[i] = pair_sum16(pg[i], pg[H + i]);
#pragma unroll
                        for (int i = 0; i < Q; ++i)
                            s_red[s][wave][2 * DKP + c * E + h * H + h2 * Q + i] = pair_sum32(P[i], P[Q + i]);
                    } else {
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            float x = pg[e] + lane_xor16(pg[e]);
                            x += lane_xor32(x);
                            if (gw == 0) s_red[s][wave][2 * DKP + c * E + e] = x;
                        }
                    }
                }
            }
            __syncthreads();
            // Write this workgroup's partial sums for tokens [ss, ss+n), four channels per thread and step (the
            // index split has compile-time divisors); 16-byte stores when the rows allow them.
            {
                constexpr int NJ4 = DKP / 4, PER_S = NQ * NJ4;
                const size_t tok0 = (((size_t)rb * B + b) * T + ss) * Hv + hv;
                for (int i = tid; i < CS * PER_S; i += NT) {
                    const int s = i / PER_S, rem = i - s * PER_S, which = rem / NJ4, j = 4 * (rem - which * NJ4);
                    if (s < n && j < Dk) {
                        const int o = which * DKP + j;
                        // the waves' sums, added pairwise in a fixed tree: ((w0 + w1) + (w2 + w3)) + ...
                        float4 w[NW];
#pragma unroll
                        for (int u = 0; u < NW; ++u) w[u] = *reinterpret_cast<const float4 *>(&s_red[s][u][o]);
#pragma unroll
                        for (int h = 1; h < NW; h *= 2)
#pragma unroll
                            for (int u = 0; u < NW; u += 2 * h)
                                w[u] = make_float4(w[u].x + w[u + h].x, w[u].y + w[u + h].y, w[u].z + w[u + h].z,
                                                   w[u].w + w[u + h].w);
                        const float4 sum = w[0];
                        const size_t tok = tok0 + (size_t)s * Hv;
                        float *dst = which < 2 ? a.part_qk + tok * 2 * Dk + which * Dk + j : a.part_gv + tok * Dk + j;
                        if (part_vec) {
                            *reinterpret_cast<float4 *>(dst) = sum;
                        } else {
                            const float v4[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
                            for (int u = 0; u < 4; ++u)
                                if (j + u < Dk) dst[u] = v4[u];
                        }
                    }
                }
            }
            for (int i = tid; i < n * R; i += NT) {
                const int s = i / R, r = i - s * R, rr = rb * R + r;
                if (rr < Dv)
                    store_from_f32(a.dv, (((size_t)b * T + ss + s) * Hv + hv) * Dv + rr, s_row[s][r][0],
                                   a.grad_dt);
            }
            if (tid < n) {
                const int s = tid;
                float db = 0.f, dg = 0.f;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    db += s_row[s][r][1];
                    dg += s_row[s][r][2];
                }
                const size_t tok = (((size_t)rb * B + b) * T + ss + s) * Hv + hv;
                a.part_gb[tok * 2 + 0] = db;
                a.part_gb[tok * 2 + 1] = dg;
            }
        }
    }
    if (a.dstate0 && row_ok) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int j = c * E + e;
            if (j < Dk) a.dstate0[row_off + j] = dS[e];
        }
    }
}

// Sum the per-row-block partials over row blocks and over the value heads of each key head.
__global__ __launch_bounds__(256) void rec_bwd_reduce_qk(RecBwdArgs a) {
    const size_t total = (size_t)a.B * a.T * a.Hk * a.Dk;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int j = (int)(i % a.Dk);
    const size_t bth = i / a.Dk;
    const int hk = (int)(bth % a.Hk);
    const size_t bt = bth / a.Hk;
    const int rep = a.Hv / a.Hk;
    const size_t BT = (size_t)a.B * a.T;
    float sq = 0.f, sk = 0.f;
    for (int rb = 0; rb < a.nrb; ++rb) {
        for (int r = 0; r < rep; ++r) {
            const size_t tok = ((size_t)rb * BT + bt) * a.Hv + hk * rep + r;
            sq += a.part_qk[tok * 2 * a.Dk + j];
            sk += a.part_qk[tok * 2 * a.Dk + a.Dk + j];
        }
    }
    store_from_f32(a.dq, i, sq, a.grad_dt);
    store_from_f32(a.dk, i, sk, a.grad_dt);
}

__global__ __launch_bounds__(256) void rec_bwd_reduce_gates(RecBwdArgs a) {
    const size_t BT = (size_t)a.B * a.T;
    const size_t total = BT * a.Hv * (gate_vec(a.gate) ? a.Dk : 1);
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    if (gate_vec(a.gate)) {
        float s = 0.f;
        for (int rb = 0; rb < a.nrb; ++rb) s += a.part_gv[(size_t)rb * BT * a.Hv * a.Dk + i];
        a.dg[i] = a.gate == GATE_LOG_VEC ? s * expf(a.g[i]) : s;
        if (i % a.Dk == 0) {
            const size_t tok = i / a.Dk;
            float db = 0.f;
            for (int rb = 0; rb < a.nrb; ++rb) db += a.part_gb[((size_t)rb * BT * a.Hv + tok) * 2];
            a.dbeta[tok] = db;
        }
        return;
    }
    float db = 0.f, dg = 0.f;
    for (int rb = 0; rb < a.nrb; ++rb) {
        const size_t tok = (size_t)rb * BT * a.Hv + i;
        db += a.part_gb[tok * 2 + 0];
        dg += a.part_gb[tok * 2 + 1];
    }
    if (a.gate == GATE_LOG) dg *= expf(a.g[i]);
    a.dbeta[i] = db;
    a.dg[i] = dg;
}

// Dk % 4 == 0 and 16-byte aligned buffers: four channels per thread (float4 partial loads, the row blocks and value
// heads summed in the same order as above), a workgroup over 256 / (Dk / 4) token rows of one key head (grid.y).
__global__ __launch_bounds__(256) void rec_bwd_reduce_qk_vec4(RecBwdArgs a) {
    const int Dk4 = a.Dk >> 2, per = 256 / Dk4, hk = blockIdx.y;
    const int tl = threadIdx.x / Dk4, j4 = threadIdx.x - tl * Dk4;
    const size_t BT = (size_t)a.B * a.T, bt = (size_t)blockIdx.x * per + tl;
    if (tl >= per || bt >= BT) return;
    const int rep = a.Hv / a.Hk;
    float4 sq = make_float4(0.f, 0.f, 0.f, 0.f), sk = sq;
    for (int rb = 0; rb < a.nrb; ++rb) {
        for (int r = 0; r < rep; ++r) {
            const size_t tok = ((size_t)rb * BT + bt) * a.Hv + hk * rep + r;
            const float4 *p = reinterpret_cast<const float4 *>(a.part_qk + tok * 2 * a.Dk) + j4;
            const float4 x = p[0], y = p[Dk4];
            sq = make_float4(sq.x + x.x, sq.y + x.y, sq.z + x.z, sq.w + x.w);
            sk = make_float4(sk.x + y.x, sk.y + y.y, sk.z + y.z, sk.w + y.w);
        }
    }
    const size_t i = (bt * a.Hk + hk) * a.Dk + 4 * j4;
    store4_from_f32(a.dq, i, sq, a.grad_dt);
    store4_from_f32(a.dk, i, sk, a.grad_dt);
}

// Per-channel gates with Dk % 4 == 0 and 16-byte aligned rows: four channels per thread (float4 loads and
// stores, the row blocks summed in the same order as above), a workgroup over 256 / (Dk / 4) token-heads.
__global__ __launch_bounds__(256) void rec_bwd_reduce_gates_vec4(RecBwdArgs a) {
    const int Dk4 = a.Dk >> 2, per = 256 / Dk4;
    const int tl = threadIdx.x / Dk4, j4 = threadIdx.x - tl * Dk4;
    const size_t N = (size_t)a.B * a.T * a.Hv, th = (size_t)blockIdx.x * per + tl;
    if (tl >= per || th >= N) return;
    const size_t plane4 = N * (size_t)Dk4;  // one row block's partials, in float4
    const float4 *src = reinterpret_cast<const float4 *>(a.part_gv) + th * Dk4 + j4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int rb = 0; rb < a.nrb; ++rb) {
        const float4 p = src[(size_t)rb * plane4];
        s = make_float4(s.x + p.x, s.y + p.y, s.z + p.z, s.w + p.w);
    }
    if (a.gate == GATE_LOG_VEC) {  // d/d(log decay) = d/d(decay) * decay
        const float4 g = reinterpret_cast<const float4 *>(a.g)[th * Dk4 + j4];
        s = make_float4(s.x * expf(g.x), s.y * expf(g.y), s.z * expf(g.z), s.w * expf(g.w));
    }
    reinterpret_cast<float4 *>(a.dg)[th * Dk4 + j4] = s;
    if (j4 == 0) {
        float db = 0.f;
        for (int rb = 0; rb < a.nrb; ++rb) db += a.part_gb[((size_t)rb * N + th) * 2];
        a.dbeta[th] = db;
    }
}

// ---------------------------------------------------------------------------------------------------- dispatch

int pick_lane_width(int Dk) {
    if (Dk <= 16) return 1;
    if (Dk <= 32) return 2;
    if (Dk <= 64) return 4;
    if (Dk <= 128) return 8;
    if (Dk <= 256) return 16;
    return 0;
}

int rec_num_row_blocks(int Dv) { return (Dv + ROWS - 1) / ROWS; }

// Value rows per backward workgroup.  32 (8 waves) halves the per-row-block partial sums that rec_bwd writes and
// rec_bwd_reduce_* read back, but one 8-wave workgroup per CU leaves every SIMD waiting at its barriers where two
// 4-wave ones overlap: at B=4, T=4096, Hv=32 it made rec_bwd 0.8 ms slower for 0.45 ms less reduction with scalar
// gates, and 0.55 ms slower for 0.85 ms less with per-channel gates (whose dg partials double the traffic).  So 32
// is taken for per-channel gates only, when the grid keeps at least 512 workgroups (two rounds of one per CU) and
// up to Dk = 128 (the 8-wave LDS sums of wider rows would not fit); 16 (4 waves) otherwise.
int rec_bwd_rows(int B, int Hv, int Dk, int Dv, int gate) {
    if (!gate_vec(gate) || pick_lane_width(Dk) > 8 || Dv <= ROWS) return ROWS;
    return (int64_t)B * Hv * ((Dv + 2 * ROWS - 1) / (2 * ROWS)) >= 512 ? 2 * ROWS : ROWS;
}

int rec_bwd_row_blocks(int B, int Hv, int Dk, int Dv, int gate) {
    const int r = rec_bwd_rows(B, Hv, Dk, Dv, gate);
    return (Dv + r - 1) / r;
}

int rec_max_sub(int T, int chunk) {
    const int span = chunk < T ? chunk : T;
    const int ns = (span + BWD_CS - 1) / BWD_CS - 1;
    return ns > 0 ? ns : 0;
}

size_t rec_sub_floats(int B, int Hv, int Dk, int Dv, int T, int chunk, int gate) {
    const int E = pick_lane_width(Dk);
    return (size_t)B * Hv * rec_bwd_row_blocks(B, Hv, Dk, Dv, gate) * rec_max_sub(T, chunk) *
           rec_bwd_rows(B, Hv, Dk, Dv, gate) * 16 * E;
}

template <int E, int DT>
static void launch_fwd_et(const RecFwdArgs &a, hipStream_t st) {
    dim3 grid(rec_num_row_blocks(a.Dv), a.Hv, a.B);
    const bool vec = gate_vec(a.gate), masked = a.mask != nullptr;
    if (vec && masked) hipLaunchKernelGGL((rec_fwd_kernel<E, true, DT, true>), grid, dim3(THREADS), 0, st, a);
    else if (vec) hipLaunchKernelGGL((rec_fwd_kernel<E, true, DT, false>), grid, dim3(THREADS), 0, st, a);
    else if (masked) hipLaunchKernelGGL((rec_fwd_kernel<E, false, DT, true>), grid, dim3(THREADS), 0, st, a);
    else hipLaunchKernelGGL((rec_fwd_kernel<E, false, DT, false>), grid, dim3(THREADS), 0, st, a);
}

template <int E>
static void launch_fwd_e(const RecFwdArgs &a, hipStream_t st) {
    // bf16 and fp32 fixed at compile time; fp16 read from the arguments
    if (a.in_dt == DT_BF16) launch_fwd_et<E, DT_BF16>(a, st);
    else if (a.in_dt == DT_F32) launch_fwd_et<E, DT_F32>(a, st);
    else launch_fwd_et<E, -1>(a, st);
}

template <int E>
static void launch_decode_e(const RecFwdArgs &a, hipStream_t st) {
    const dim3 grid(rec_num_row_blocks(a.Dv), a.Hv, a.B);
    const bool vec = gate_vec(a.gate);
    if (a.in_dt == DT_BF16) {
        if (vec) hipLaunchKernelGGL((rec_decode_kernel<E, true, DT_BF16>), grid, dim3(THREADS), 0, st, a);
        else hipLaunchKernelGGL((rec_decode_kernel<E, false, DT_BF16>), grid, dim3(THREADS), 0, st, a);
    } else if (a.in_dt == DT_F32) {
        if (vec) hipLaunchKernelGGL((rec_decode_kernel<E, true, DT_F32>), grid, dim3(THREADS), 0, st, a);
        else hipLaunchKernelGGL((rec_decode_kernel<E, false, DT_F32>), grid, dim3(THREADS), 0, st, a);
    } else {
        if (vec) hipLaunchKernelGGL((rec_decode_kernel<E, true, -1>), grid, dim3(THREADS), 0, st, a);
        else hipLaunchKernelGGL((rec_decode_kernel<E, false, -1>), grid, dim3(THREADS), 0, st, a);
    }
}

void launch_rec_decode(const RecFwdArgs &a, hipStream_t st) {
    switch (pick_lane_width(a.Dk)) {
        case 1: launch_decode_e<1>(a, st); break;
        case 2: launch_decode_e<2>(a, st); break;
        case 4: launch_decode_e<4>(a, st); break;
        case 8: launch_decode_e<8>(a, st); break;
        default: launch_decode_e<16>(a, st); break;
    }
}

void launch_rec_fwd(const RecFwdArgs &a, hipStream_t st) {
    switch (pick_lane_width(a.Dk)) {
        case 1: launch_fwd_e<1>(a, st); break;
        case 2: launch_fwd_e<2>(a, st); break;
        case 4: launch_fwd_e<4>(a, st); break;
        case 8: launch_fwd_e<8>(a, st); break;
        default: launch_fwd_e<16>(a, st); break;
    }
}

template <int E, int DT, int NW>
static void launch_bwd_etw(const RecBwdArgs &a, hipStream_t st) {
    const dim3 grid(a.nrb, a.Hv, a.B), block(64 * NW);
    // Per-channel gates keep the mask selects even without a mask (every token then keeps its candidate): built
    // without them, that backward measured slower (11.30 against 11.02 ms at B=4, T=4096, Hv=32) although it issues
    // 12% fewer instructions.
    if (gate_vec(a.gate))
        hipLaunchKernelGGL((rec_bwd_kernel<E, true, DT, NW, true>), grid, block, 0, st, a);
    else if (a.mask)
        hipLaunchKernelGGL((rec_bwd_kernel<E, false, DT, NW, true>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((rec_bwd_kernel<E, false, DT, NW, false>), grid, block, 0, st, a);
}

template <int E, int DT>
static void launch_bwd_et(const RecBwdArgs &a, hipStream_t st) {
    if constexpr (E <= 8) {
        if (rec_bwd_rows(a.B, a.Hv, a.Dk, a.Dv, a.gate) == 2 * ROWS) return launch_bwd_etw<E, DT, 8>(a, st);
    }
    launch_bwd_etw<E, DT, 4>(a, st);
}

// inputs and cotangent both bf16 or both fp32: fixed at compile time; fp16 or mixed (e.g. a wider cotangent): read
// at run time
template <int E>
static void launch_bwd_e(const RecBwdArgs &a, hipStream_t st) {
    if (a.in_dt == a.dy_dt && a.in_dt == DT_BF16) launch_bwd_et<E, DT_BF16>(a, st);
    else if (a.in_dt == a.dy_dt && a.in_dt == DT_F32) launch_bwd_et<E, DT_F32>(a, st);
    else launch_bwd_et<E, -1>(a, st);
}

void launch_rec_bwd(const RecBwdArgs &a, hipStream_t st) {
    switch (pick_lane_width(a.Dk)) {
        case 1: launch_bwd_e<1>(a, st); break;
        case 2: launch_bwd_e<2>(a, st); break;
        case 4: launch_bwd_e<4>(a, st); break;
        case 8: launch_bwd_e<8>(a, st); break;
        default: launch_bwd_e<16>(a, st); break;
    }
}

void launch_rec_bwd_reduce(const RecBwdArgs &a, hipStream_t st) {
    const size_t nqk = (size_t)a.B * a.T * a.Hk * a.Dk;
    const size_t ng = (size_t)a.B * a.T * a.Hv * (gate_vec(a.gate) ? a.Dk : 1);
    const bool qk4 = (a.Dk & 3) == 0 && ((reinterpret_cast<uintptr_t>(a.part_qk) | reinterpret_cast<uintptr_t>(a.dq) |
                                          reinterpret_cast<uintptr_t>(a.dk)) & 15) == 0;
    if (nqk && qk4) {
        const int per = 256 / (a.Dk >> 2);
        const size_t BT = (size_t)a.B * a.T;
        hipLaunchKernelGGL(rec_bwd_reduce_qk_vec4, dim3((unsigned)((BT + per - 1) / per), a.Hk), dim3(256), 0, st,
                           a);
    } else if (nqk) {
        hipLaunchKernelGGL(rec_bwd_reduce_qk, dim3((unsigned)((nqk + 255) / 256)), dim3(256), 0, st, a);
    }
    if (!ng) return;
    const bool aligned = ((reinterpret_cast<uintptr_t>(a.part_gv) | reinterpret_cast<uintptr_t>(a.dg) |
                           reinterpret_cast<uintptr_t>(a.g)) & 15) == 0;
    const bool vec4 = gate_vec(a.gate) && (a.Dk & 3) == 0 && aligned;
    if (vec4) {
        const size_t N = (size_t)a.B * a.T * a.Hv;
        const int per = 256 / (a.Dk >> 2);
        hipLaunchKernelGGL(rec_bwd_reduce_gates_vec4, dim3((unsigned)((N + per - 1) / per)), dim3(256), 0, st, a);
    } else {
        hipLaunchKernelGGL(rec_bwd_reduce_gates, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, st, a);
    }
}

}  // namespace gdn
