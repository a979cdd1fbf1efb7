// Streaming kernels that surround the GDN recurrence inside one block, for gfx950:
//   gates (log decay + beta), q/k L2 norm, causal depthwise conv1d + SiLU, gated RMSNorm * SiLU(z),
// each with its backward.  All of them are HBM-bound elementwise/row work:
//   * every input element is read once with 8- or 16-byte vector loads, every output written once;
//   * per-row reductions (L2 norm, RMS) stay inside a group of L lanes of one wavefront (xor shuffles);
//   * parameter gradients (dA_log, ddt_bias, conv weights, norm weight) are reduced deterministically:
//     per-workgroup partials in a fixed order, then a fixed-order column sum.  No atomics.
//
// Specs: engine/include/gdn.h:7-25 (conv step, l2norm, gates), engine/include/ops.h:7-11 and
// engine/src/gdn_layer.c:35-55 (per-head L2 norm scales, gated RMSNorm).
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {
namespace ops {

constexpr int NT = 256;

// 1 / (1 + 2^(-x log2(e))) on v_exp_f32 and v_rcp_f32 (about 2 ulp); 0 and 1 at the ends, NaN stays NaN
__device__ __forceinline__ float sigmoidf_(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// softplus(t) = t > 20 ? t : log1p(exp(t))   (engine/include/gdn.h:23-24)
__device__ __forceinline__ float softplus_(float t) { return t > 20.f ? t : log1pf(expf(t)); }

// Sum over aligned groups of L lanes (every lane of the wave active); all lanes of a group get the same bits.
template <int L>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(L == 1 || L == 2 || L == 4 || L == 8 || L == 16 || L == 32 || L == 64, "L is a power of two");
    if constexpr (L >= 2) x += dpp_mov<DPP_QUAD_1032>(x);
    if constexpr (L >= 4) x += dpp_mov<DPP_QUAD_2301>(x);
    if constexpr (L >= 8) x += dpp_mov<DPP_ROW_HALF_MIRROR>(x);
    if constexpr (L >= 16) x += dpp_mov<DPP_ROW_MIRROR>(x);
    if constexpr (L >= 32) x += lane_xor16(x);
    if constexpr (L >= 64) x += lane_xor32(x);
    return x;
}

__device__ __forceinline__ float half_bits_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu)));
}

// V consecutive elements starting at element i (i % V == 0, buffer base 16-byte aligned).
template <int V>
__device__ __forceinline__ void loadv(const void *p, size_t i, int dt, float (&o)[V]) {
    if constexpr (V == 1) {
        o[0] = load_as_f32(p, i, dt);
    } else if constexpr (V == 4) {
        if (dt == DT_F32) {
            const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
            o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        } else {
            const uint2 u = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(p) + i);
            const uint32_t w[2] = {u.x, u.y};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (dt == DT_BF16) {
                    o[2 * j] = __uint_as_float(w[j] << 16);
                    o[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
                } else {
                    o[2 * j] = half_bits_to_f32(w[j]);
                    o[2 * j + 1] = half_bits_to_f32(w[j] >> 16);
                }
            }
        }
    } else {
        static_assert(V == 8, "V is 1, 4 or 8");
        if (dt == DT_F32) {
            const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
            const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i + 4);
            o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
            o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
        } else {
            const uint4 u = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + i);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (dt == DT_BF16) {
                    o[2 * j] = __uint_as_float(w[j] << 16);
                    o[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
                } else {
                    o[2 * j] = half_bits_to_f32(w[j]);
                    o[2 * j + 1] = half_bits_to_f32(w[j] >> 16);
                }
            }
        }
    }
}

__device__ __forceinline__ uint32_t pack2(float a, float b, int dt) {
    if (dt == DT_BF16) return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
    return (uint32_t)__half_as_ushort(__float2half(a)) | ((uint32_t)__half_as_ushort(__float2half(b)) << 16);
}

template <int V>
__device__ __forceinline__ void storev(void *p, size_t i, int dt, const float (&o)[V]) {
    if constexpr (V == 1) {
        store_from_f32(p, i, o[0], dt);
    } else if constexpr (V == 4) {
        if (dt == DT_F32) {
            *reinterpret_cast<float4 *>(static_cast<float *>(p) + i) = make_float4(o[0], o[1], o[2], o[3]);
        } else {
            *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p) + i) =
                make_uint2(pack2(o[0], o[1], dt), pack2(o[2], o[3], dt));
        }
    } else {
        static_assert(V == 8, "V is 1, 4 or 8");
        if (dt == DT_F32) {
            *reinterpret_cast<float4 *>(static_cast<float *>(p) + i) = make_float4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<float4 *>(static_cast<float *>(p) + i + 4) = make_float4(o[4], o[5], o[6], o[7]);
        } else {
            *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(p) + i) =
                make_uint4(pack2(o[0], o[1], dt), pack2(o[2], o[3], dt), pack2(o[4], o[5], dt),
                           pack2(o[6], o[7], dt));
        }
    }
}

// ------------------------------------------------------------------------------------------- column sums

// s_j = sum_r part[r * ncols + j] (r ascending), written to out[j] for j < split and out2[j - split] after.
__device__ __forceinline__ void put_col(float *out, float *out2, int split, int j, float s) {
    if (j < split)
        out[j] = s;
    else
        out2[j - split] = s;
}

// One thread per column: for few partial rows.
__global__ void colsum_thread_kernel(const float *part, int nrows, int ncols, float *out, float *out2, int split) {
    const int j = blockIdx.x * NT + threadIdx.x;
    if (j >= ncols) return;
    float s = 0.f;
    for (int r = 0; r < nrows; ++r) s += part[(size_t)r * ncols + j];
    put_col(out, out2, split, j, s);
}

// One workgroup per column: thread t sums rows t, t+NT, ... in order, then a fixed tree over the threads.
__global__ __launch_bounds__(NT) void colsum_block_kernel(const float *part, int nrows, int ncols, float *out,
                                                          float *out2, int split) {
    __shared__ float red[NT];
    const int j = blockIdx.x, tid = threadIdx.x;
    float s = 0.f;
    for (int r = tid; r < nrows; r += NT) s += part[(size_t)r * ncols + j];
    red[tid] = s;
    __syncthreads();
#pragma unroll
    for (int h = NT / 2; h >= 1; h >>= 1) {
        if (tid < h) red[tid] += red[tid + h];
        __syncthreads();
    }
    if (tid == 0) put_col(out, out2, split, j, red[0]);
}

// ------------------------------------------------------------------------------------------------ gates

// g = -exp(A_log[h]) softplus(a + dt_bias[h]) as log decay (log_space) or decay exp(g); beta = s sigmoid(b)
__global__ __launch_bounds__(NT) void gates_fwd_kernel(const void *a, const void *b, const float *A_log,
                                                       const float *dt_bias, float *g, float *beta, size_t n,
                                                       int Hv, int in_dt, int log_space, float beta_scale) {
    const size_t i = (size_t)blockIdx.x * NT + threadIdx.x;
    if (i >= n) return;
    const int h = (int)(i % Hv);
    const float x = load_as_f32(a, i, in_dt) + dt_bias[h];
    const float gl = -expf(A_log[h]) * softplus_(x);
    g[i] = log_space ? gl : expf(gl);
    beta[i] = beta_scale * sigmoidf_(load_as_f32(b, i, in_dt));
}

// da, db elementwise and per-workgroup partials of dA_log / ddt_bias.  A workgroup owns GATE_TOK tokens x
// all Hv heads (Hv <= NT); thread tid handles head tid % Hv for tokens slot, slot + nslot, ...
constexpr int GATE_TOK = 32;
__global__ __launch_bounds__(NT) void gates_bwd_kernel(const void *a, const void *b, const float *A_log,
                                                       const float *dt_bias, const float *g, const float *dg,
                                                       const float *dbeta, void *da, void *db, float *part,
                                                       size_t tokens, int Hv, int in_dt, int grad_dt, int log_space,
                                                       float beta_scale) {
    __shared__ float sA[NT], sT[NT];
    const int tid = threadIdx.x;
    const size_t tok0 = (size_t)blockIdx.x * GATE_TOK;
    const int ntok = (int)min((size_t)GATE_TOK, tokens - tok0);
    const int nslot = NT / Hv;
    const int h = tid % Hv, slot = tid / Hv;
    float accA = 0.f, accT = 0.f;
    if (slot < nslot) {
        const float e = expf(A_log[h]), bias = dt_bias[h];
        for (int t = slot; t < ntok; t += nslot) {
            const size_t i = (tok0 + t) * Hv + h;
            const float x = load_as_f32(a, i, in_dt) + bias;
            const float gv = g[i];
            const float gl = log_space ? gv : -e * softplus_(x);
            const float dgl = log_space ? dg[i] : dg[i] * gv;  // gradient w.r.t. the log decay
            const float dx = dgl * -e * (x > 20.f ? 1.f : sigmoidf_(x));
            store_from_f32(da, i, dx, grad_dt);
            accA = fmaf(dgl, gl, accA);  // d(log decay)/dA_log = log decay
            accT += dx;
            const float sb = sigmoidf_(load_as_f32(b, i, in_dt));
            store_from_f32(db, i, dbeta[i] * beta_scale * sb * (1.f - sb), grad_dt);
        }
    }
    sA[tid] = accA;
    sT[tid] = accT;
    __syncthreads();
    if (tid < Hv) {
        float s1 = 0.f, s2 = 0.f;
        for (int s = 0; s < nslot; ++s) {
            s1 += sA[s * Hv + tid];
            s2 += sT[s * Hv + tid];
        }
        part[(size_t)blockIdx.x * 2 * Hv + tid] = s1;
        part[(size_t)blockIdx.x * 2 * Hv + Hv + tid] = s2;
    }
}

// ------------------------------------------------------------------------------------------------ l2 norm

// L lanes per row, 8 elements per lane (D = 8L); NT / L rows per workgroup.
// y = scale * x / sqrt(sum x^2 + eps)
template <int L>
__global__ __launch_bounds__(NT) void l2norm_fwd_vec(const void *x, void *y, size_t rows, float eps, float scale,
                                                     int dt) {
    const size_t row = (size_t)blockIdx.x * (NT / L) + threadIdx.x / L;
    if (row >= rows) return;
    const size_t base = row * (8 * L) + (threadIdx.x % L) * 8;
    float v[8];
    loadv<8>(x, base, dt, v);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
    const float inv = scale * rsqrtf(group_sum<L>(ss) + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= inv;
    storev<8>(y, base, dt, v);
}

// dx = s/n (dy - x (x . dy) / n^2),  n = sqrt(sum x^2 + eps)
template <int L>
__global__ __launch_bounds__(NT) void l2norm_bwd_vec(const void *x, const void *dy, void *dx, size_t rows, float eps,
                                                     float scale, int dt, int dy_dt) {
    const size_t row = (size_t)blockIdx.x * (NT / L) + threadIdx.x / L;
    if (row >= rows) return;
    const size_t base = row * (8 * L) + (threadIdx.x % L) * 8;
    float v[8], d[8];
    loadv<8>(x, base, dt, v);
    loadv<8>(dy, base, dy_dt, d);
    float ss = 0.f, xd = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        ss = fmaf(v[j], v[j], ss);
        xd = fmaf(v[j], d[j], xd);
    }
    const float n2 = group_sum<L>(ss) + eps, dot = group_sum<L>(xd);
    const float c1 = scale * rsqrtf(n2), c2 = c1 * dot / n2;
#pragma unroll
    for (int j = 0; j < 8; ++j) d[j] = c1 * d[j] - c2 * v[j];
    storev<8>(dx, base, dt, d);
}

// Any D: one wavefront per row.
__global__ __launch_bounds__(NT) void l2norm_fwd_any(const void *x, void *y, size_t rows, int D, float eps,
                                                     float scale, int dt) {
    const size_t row = (size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = row * D;
    float ss = 0.f;
    for (int j = l; j < D; j += 64) {
        const float v = load_as_f32(x, base + j, dt);
        ss = fmaf(v, v, ss);
    }
    const float inv = scale * rsqrtf(group_sum<64>(ss) + eps);
    for (int j = l; j < D; j += 64) store_from_f32(y, base + j, load_as_f32(x, base + j, dt) * inv, dt);
}

__global__ __launch_bounds__(NT) void l2norm_bwd_any(const void *x, const void *dy, void *dx, size_t rows, int D,
                                                     float eps, float scale, int dt, int dy_dt) {
    const size_t row = (size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = row * D;
    float ss = 0.f, xd = 0.f;
    for (int j = l; j < D; j += 64) {
        const float v = load_as_f32(x, base + j, dt), d = load_as_f32(dy, base + j, dy_dt);
        ss = fmaf(v, v, ss);
        xd = fmaf(v, d, xd);
    }
    const float n2 = group_sum<64>(ss) + eps, dot = group_sum<64>(xd);
    const float c1 = scale * rsqrtf(n2), c2 = c1 * dot / n2;
    for (int j = l; j < D; j += 64) {
        const float v = load_as_f32(x, base + j, dt), d = load_as_f32(dy, base + j, dy_dt);
        store_from_f32(dx, base + j, c1 * d - c2 * v, dt);
    }
}

// ------------------------------------------------------------------------------------------------ conv1d + SiLU

// Causal depthwise conv over time + SiLU (engine/include/gdn.h:7-15 over a whole sequence), optionally fused
// with the q/k/v split and the per-head L2 norm of q and k (engine/src/gdn_layer.c:29-39):
//   c[t, ch] = silu(sum_j w[ch*K + j] x[t - (K-1) + j, ch])      ch < C = 2*qk + nv
//   channels [0, qk) are q, [qk, 2qk) k, [2qk, C) v; with L > 0 each head of Dk = L*V q/k channels is scaled by
//   (scale_q for q, 1 for k) / sqrt(sum c^2 + eps) and q, k, v are written to separate contiguous tensors
//   ([.., qk], [.., qk], [.., nv] per token).  With qk = 0 this is the plain conv: v is the [B,T,C] output.
// A workgroup is 4 wavefronts stacked in time: wavefront s covers tokens [t0 + s*CONV_TT, +CONV_TT) and every
// lane V consecutive channels (16-byte loads: V = 8 for 16-bit data, 4 for fp32).  Each thread walks its
// tokens in order keeping the last K-1 inputs in registers, so an input is read once (plus a K-1 token halo per
// CONV_TT tokens); U tokens are loaded ahead per step to keep several loads in flight per lane.  The L lanes of
// one q/k head reduce with xor shuffles (heads align with lane groups because 64V is a multiple of Dk).
constexpr int CONV_TT = 64;
constexpr int CONV_SLICES = NT / 64;

struct ConvArgs {
    const void *x;          // [B][T][C]
    const float *w;         // [C][K]
    const float *state_in;  // [B][K-1][C] fp32 or null (zeros)
    void *q, *k, *v;        // forward outputs / backward cotangents: [B][T][qk], [B][T][qk], [B][T][C - 2qk]
    void *dx;               // backward output [B][T][C]
    float *part;            // backward dw partials [B * ntiles][C][K]
    int T, C, qk, dt, g_dt; // g_dt: dtype of q/k/v (the cotangents' dtype in the backward)
    float scale_q, eps;
};

// x at token t (t < 0: the carried conv state, zero when absent; t >= T: zero)
template <int K, int V>
__device__ __forceinline__ void conv_x(const void *x, const float *state_in, int b, int t, int T, int C, int c0,
                                       int dt, float (&o)[V]) {
    if (t >= 0 && t < T) {
        loadv<V>(x, ((size_t)b * T + t) * C + c0, dt, o);
    } else if (t < 0 && state_in) {
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] = state_in[((size_t)b * (K - 1) + (t + K - 1)) * C + c0 + v];
    } else {
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] = 0.f;
    }
}

// x at token t of the token loop (0 <= t; t >= tend reads as zero) without a branch: the load goes to a clamped
// token and a select zeroes it, so the loads of several tokens stay in flight together.
template <int V>
__device__ __forceinline__ void conv_x_in(const void *x, int b, int t, int tend, int T, int C, int c0, int dt,
                                          float (&o)[V]) {
    const bool ok = t < tend;
    float r[V];
    loadv<V>(x, ((size_t)b * T + (ok ? t : tend - 1)) * C + c0, dt, r);
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = ok ? r[v] : 0.f;
}

// Where channel c0 of a token lives in the split q/k/v tensors: base pointer, row length, column; region 0/1/2.
struct SplitPos {
    void *base;
    int row, col, region;
};
__device__ __forceinline__ SplitPos split_pos(const ConvArgs &a, int c0) {
    if (c0 < a.qk) return {a.q, a.qk, c0, 0};
    if (c0 < 2 * a.qk) return {a.k, a.qk, c0 - a.qk, 1};
    return {a.v, a.C - 2 * a.qk, c0 - 2 * a.qk, 2};
}

// DT >= 0: x and q/k/v are all of that dtype, known at compile time (the loads and stores of the token loop then
// carry no dtype branches, which would make the compiler wait for every load where the branches join); DT < 0:
// the dtypes are read from the arguments.
template <int K, int V, int U, int L, int DT>
__global__ __launch_bounds__(NT) void conv_fwd_kernel(ConvArgs a) {
    const int dt = DT >= 0 ? DT : a.dt;
    const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
    const int c0 = (blockIdx.x * 64 + lane) * V;
    const int t0 = (blockIdx.y * CONV_SLICES + slice) * CONV_TT, b = blockIdx.z;
    const int T = a.T, C = a.C;
    if (t0 >= T) return;  // uniform over the wavefront
    const bool active = c0 < C;  // lanes past C only take part in the head shuffles (v region, unused)
    const int cc = active ? c0 : 0;
    const SplitPos sp = split_pos(a, cc);
    const float nscale = sp.region == 0 ? a.scale_q : 1.f;
    float wk[K][V], hist[K - 1][V];
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
        for (int j = 0; j < K; ++j) wk[j][v] = a.w[(size_t)(cc + v) * K + j];
#pragma unroll
    for (int j = 0; j < K - 1; ++j) conv_x<K, V>(a.x, a.state_in, b, t0 - (K - 1) + j, T, C, cc, dt, hist[j]);
    const int t1 = min(T, t0 + CONV_TT);
    for (int t = t0; t < t1; t += U) {
        float xs[U][V];
#pragma unroll
        for (int u = 0; u < U; ++u) conv_x_in<V>(a.x, b, t + u, t1, T, C, cc, dt, xs[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (t + u >= t1) break;
            float o[V], ss = 0.f;
#pragma unroll
            for (int v = 0; v < V; ++v) {
                float pre = wk[K - 1][v] * xs[u][v];
#pragma unroll
                for (int j = 0; j < K - 1; ++j) pre = fmaf(wk[j][v], hist[j][v], pre);
#pragma unroll
                for (int j = 0; j + 1 < K - 1; ++j) hist[j][v] = hist[j + 1][v];
                hist[K - 2][v] = xs[u][v];
                o[v] = pre * sigmoidf_(pre);
                ss = fmaf(o[v], o[v], ss);
            }
            if constexpr (L > 0) {
                ss = group_sum<L>(ss);
                if (sp.region < 2) {
                    const float inv = nscale * rsqrtf(ss + a.eps);
#pragma unroll
                    for (int v = 0; v < V; ++v) o[v] *= inv;
                }
            }
            if (active) storev<V>(sp.base, ((size_t)b * T + t + u) * sp.row + sp.col, dt, o);
        }
    }
}

// The last K-1 inputs after the sequence, oldest first: state_out[b][j][c] = x at T-(K-1)+j (from state_in when
// that is before the sequence).  state_out must not alias state_in.
__global__ void conv_state_kernel(const void *x, const float *state_in, float *state_out, int B, int T, int C, int K,
                                  int dt) {
    const size_t i = (size_t)blockIdx.x * NT + threadIdx.x;
    if (i >= (size_t)B * (K - 1) * C) return;
    const int c = (int)(i % C), j = (int)((i / C) % (K - 1)), b = (int)(i / ((size_t)C * (K - 1)));
    const int t = T - (K - 1) + j;
    float val = 0.f;
    if (t >= 0)
        val = load_as_f32(x, ((size_t)b * T + t) * C + c, dt);
    else if (state_in)
        val = state_in[((size_t)b * (K - 1) + (t + K - 1)) * C + c];
    state_out[i] = val;
}

// Backward, in scatter form.  For each token t (in order) the thread rebuilds pre[t] from its window of K inputs,
// turns the cotangent of the (normalised) output into dpre[t] = dc silu'(pre), adds dpre[t] x[t-(K-1)+j] to
// dw[j] and w[j] dpre[t] to the running dx of token t-(K-1)+j; dx of token t-(K-1) is then complete and stored.
// The thread runs K-1 tokens past its tile so its last dx values receive their full sums (those halo tokens add
// nothing to dw).  L2 norm backward per q/k head: dc = s/n (g - c (c.g)/n^2), n^2 = sum c^2 + eps.
// dw partials of the workgroup (its 4 time slices summed in order) go to
// part[(b * gridDim.y + blockIdx.y) * C*K + c*K + j].
template <int K, int V, int U, int L, int DT>
__global__ __launch_bounds__(NT) void conv_bwd_kernel(ConvArgs a) {
    __shared__ float red[CONV_SLICES][64 * V * K];
    const int dt = DT >= 0 ? DT : a.dt, gdt = DT >= 0 ? DT : a.g_dt;
    const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
    const int c0 = (blockIdx.x * 64 + lane) * V;
    const int t0 = (blockIdx.y * CONV_SLICES + slice) * CONV_TT, b = blockIdx.z;
    const int T = a.T, C = a.C;
    const bool active = c0 < C;
    float dwp[K][V];
#pragma unroll
    for (int j = 0; j < K; ++j)
#pragma unroll
        for (int v = 0; v < V; ++v) dwp[j][v] = 0.f;
    if (t0 < T) {  // uniform over the wavefront
        const int cc = active ? c0 : 0;
        const SplitPos sp = split_pos(a, cc);
        const float nscale = sp.region == 0 ? a.scale_q : 1.f;
        float wk[K][V], xw[K][V], acc[K][V];
#pragma unroll
        for (int v = 0; v < V; ++v)
#pragma unroll
            for (int j = 0; j < K; ++j) {
                wk[j][v] = a.w[(size_t)(cc + v) * K + j];
                acc[j][v] = 0.f;
            }
#pragma unroll
        for (int j = 0; j < K - 1; ++j) conv_x<K, V>(a.x, a.state_in, b, t0 - (K - 1) + j, T, C, cc, dt, xw[j]);
        const int t1 = min(T, t0 + CONV_TT), tend = min(T, t1 + K - 1);
        for (int t = t0; t < tend; t += U) {
            float xn[U][V], gn[U][V];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                conv_x_in<V>(a.x, b, t + u, tend, T, C, cc, dt, xn[u]);
                const bool ok = t + u < tend;
                float r[V];
                loadv<V>(sp.base, ((size_t)b * T + (ok ? t + u : tend - 1)) * sp.row + sp.col, gdt, r);
#pragma unroll
                for (int v = 0; v < V; ++v) gn[u][v] = ok ? r[v] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (t + u >= tend) break;
                float pre[V], s[V], c[V], ss = 0.f, cg = 0.f;
#pragma unroll
                for (int v = 0; v < V; ++v) {
                    xw[K - 1][v] = xn[u][v];
                    float p = 0.f;
#pragma unroll
                    for (int j = 0; j < K; ++j) p = fmaf(wk[j][v], xw[j][v], p);
                    pre[v] = p;
                    s[v] = sigmoidf_(p);
                    c[v] = p * s[v];
                    ss = fmaf(c[v], c[v], ss);
                    cg = fmaf(c[v], gn[u][v], cg);
                }
                float dc[V];
#pragma unroll
                for (int v = 0; v < V; ++v) dc[v] = gn[u][v];
                if constexpr (L > 0) {
                    ss = group_sum<L>(ss);
                    cg = group_sum<L>(cg);
                    if (sp.region < 2) {
                        const float n2 = ss + a.eps, c1 = nscale * rsqrtf(n2), c2 = c1 * cg / n2;
#pragma unroll
                        for (int v = 0; v < V; ++v) dc[v] = c1 * dc[v] - c2 * c[v];
                    }
                }
                const bool in_tile = t + u < t1;
#pragma unroll
                for (int v = 0; v < V; ++v) {
                    const float dp = dc[v] * s[v] * (1.f + pre[v] * (1.f - s[v]));
#pragma unroll
                    for (int j = 0; j < K; ++j) {
                        if (in_tile) dwp[j][v] = fmaf(dp, xw[j][v], dwp[j][v]);
                        acc[j][v] = fmaf(wk[j][v], dp, acc[j][v]);
                    }
                }
                const int ts = t + u - (K - 1);  // its dx is now complete
                if (active && ts >= t0 && ts < t1) storev<V>(a.dx, ((size_t)b * T + ts) * C + cc, dt, acc[0]);
#pragma unroll
                for (int v = 0; v < V; ++v) {
#pragma unroll
                    for (int j = 0; j + 1 < K; ++j) {
                        acc[j][v] = acc[j + 1][v];
                        xw[j][v] = xw[j + 1][v];
                    }
                    acc[K - 1][v] = 0.f;
                }
            }
        }
        // the sequence ended before the halo did: the last K-1 tokens' sums are complete (dpre past T is zero)
#pragma unroll
        for (int m = 0; m < K - 1; ++m) {
            const int ts = tend - (K - 1) + m;
            if (active && ts >= t0 && ts < t1) storev<V>(a.dx, ((size_t)b * T + ts) * C + cc, dt, acc[m]);
        }
    }
#pragma unroll
    for (int j = 0; j < K; ++j)
#pragma unroll
        for (int v = 0; v < V; ++v) red[slice][(lane * V + v) * K + j] = dwp[j][v];
    __syncthreads();
    const size_t prow = ((size_t)b * gridDim.y + blockIdx.y) * C * K;
    const int cbase = blockIdx.x * 64 * V;
    for (int e = threadIdx.x; e < 64 * V * K; e += NT) {
        if (cbase * K + e >= C * K) break;
        float s = 0.f;
#pragma unroll
        for (int sl = 0; sl < CONV_SLICES; ++sl) s += red[sl][e];
        a.part[prow + (size_t)cbase * K + e] = s;
    }
}

// ------------------------------------------------------------------------------------------------ gated RMSNorm

// out = y / sqrt(mean(y^2) + eps) * w * silu(z) per row of D = 8L   (engine/src/gdn_layer.c:47-55)
template <int L>
__global__ __launch_bounds__(NT) void grms_fwd_vec(const void *y, const void *z, const float *w, void *out,
                                                   size_t rows, float eps, int dt, int z_dt) {
    constexpr int D = 8 * L;
    const size_t row = (size_t)blockIdx.x * (NT / L) + threadIdx.x / L;
    if (row >= rows) return;
    const int col = (threadIdx.x % L) * 8;
    const size_t base = row * D + col;
    float v[8], zv[8], wv[8];
    loadv<8>(y, base, dt, v);
    loadv<8>(z, base, z_dt, zv);
    loadv<8>(w, col, DT_F32, wv);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
    const float r = rsqrtf(group_sum<L>(ss) * (1.f / D) + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * r * wv[j] * (zv[j] * sigmoidf_(zv[j]));
    storev<8>(out, base, dt, v);
}

// n = y r;  dn = dout w silu(z);  dy = r (dn - n mean(dn n));  dz = dout n w silu'(z);  dw += dout n silu(z).
// A workgroup walks GRMS_ROWS rows; each lane keeps dw for its 8 columns, the NT/L row groups are summed in
// order into part[blockIdx.x][D].
constexpr int GRMS_ROWS = 512;
template <int L>
__global__ __launch_bounds__(NT) void grms_bwd_vec(const void *y, const void *z, const float *w, const void *dout,
                                                   void *dy, void *dz, float *part, size_t rows, float eps, int dt,
                                                   int z_dt, int dout_dt) {
    constexpr int D = 8 * L, G = NT / L;
    __shared__ float red[G][D];
    const int grp = threadIdx.x / L, col = (threadIdx.x % L) * 8;
    float wv[8], dw[8];
    loadv<8>(w, col, DT_F32, wv);
#pragma unroll
    for (int j = 0; j < 8; ++j) dw[j] = 0.f;
    const size_t r0 = (size_t)blockIdx.x * GRMS_ROWS;
    for (int rr = grp; rr < GRMS_ROWS; rr += G) {
        const size_t row = r0 + rr;
        if (row >= rows) break;  // uniform across the L lanes of a row group
        const size_t base = row * D + col;
        float v[8], zv[8], go[8];
        loadv<8>(y, base, dt, v);
        loadv<8>(z, base, z_dt, zv);
        loadv<8>(dout, base, dout_dt, go);
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf(v[j], v[j], ss);
        const float r = rsqrtf(group_sum<L>(ss) * (1.f / D) + eps);
        float dn[8], sg[8], dnn = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sg[j] = sigmoidf_(zv[j]);
            v[j] *= r;  // n
            dn[j] = go[j] * wv[j] * zv[j] * sg[j];
            dnn = fmaf(dn[j], v[j], dnn);
        }
        const float mean = group_sum<L>(dnn) * (1.f / D);
        float oy[8], oz[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            oy[j] = r * (dn[j] - v[j] * mean);
            oz[j] = go[j] * v[j] * wv[j] * sg[j] * (1.f + zv[j] * (1.f - sg[j]));
            dw[j] = fmaf(go[j] * v[j], zv[j] * sg[j], dw[j]);
        }
        storev<8>(dy, base, dt, oy);
        storev<8>(dz, base, z_dt, oz);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) red[grp][col + j] = dw[j];
    __syncthreads();
    for (int j = threadIdx.x; j < D; j += NT) {
        float s = 0.f;
        for (int g = 0; g < G; ++g) s += red[g][j];
        part[(size_t)blockIdx.x * D + j] = s;
    }
}

// Any D: one wavefront per row (the backward keeps per-wavefront dw in LDS, so D <= GRMS_DMAX there).
constexpr int GRMS_DMAX = 4096;
__global__ __launch_bounds__(NT) void grms_fwd_any(const void *y, const void *z, const float *w, void *out,
                                                   size_t rows, int D, float eps, int dt, int z_dt) {
    const size_t row = (size_t)blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int l = threadIdx.x & 63;
    if (row >= rows) return;
    const size_t base = row * D;
    float ss = 0.f;
    for (int j = l; j < D; j += 64) {
        const float v = load_as_f32(y, base + j, dt);
        ss = fmaf(v, v, ss);
    }
    const float r = rsqrtf(group_sum<64>(ss) / D + eps);
    for (int j = l; j < D; j += 64) {
        const float zv = load_as_f32(z, base + j, z_dt);
        store_from_f32(out, base + j, load_as_f32(y, base + j, dt) * r * w[j] * (zv * sigmoidf_(zv)), dt);
    }
}

__global__ __launch_bounds__(NT) void grms_bwd_any(const void *y, const void *z, const float *w, const void *dout,
                                                   void *dy, void *dz, float *part, size_t rows, int D, float eps,
                                                   int dt, int z_dt, int dout_dt) {
    __shared__ float sdw[NT / 64][GRMS_DMAX];
    const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
    for (int j = l; j < D; j += 64) sdw[wv][j] = 0.f;
    const size_t r0 = (size_t)blockIdx.x * GRMS_ROWS;
    for (int rr = wv; rr < GRMS_ROWS; rr += NT / 64) {
        const size_t row = r0 + rr;
        if (row >= rows) break;
        const size_t base = row * D;
        float ss = 0.f;
        for (int j = l; j < D; j += 64) {
            const float v = load_as_f32(y, base + j, dt);
            ss = fmaf(v, v, ss);
        }
        const float r = rsqrtf(group_sum<64>(ss) / D + eps);
        float dnn = 0.f;
        for (int j = l; j < D; j += 64) {
            const float zv = load_as_f32(z, base + j, z_dt), go = load_as_f32(dout, base + j, dout_dt);
            dnn = fmaf(go * w[j] * zv * sigmoidf_(zv), load_as_f32(y, base + j, dt) * r, dnn);
        }
        const float mean = group_sum<64>(dnn) / D;
        for (int j = l; j < D; j += 64) {
            const float zv = load_as_f32(z, base + j, z_dt), go = load_as_f32(dout, base + j, dout_dt);
            const float s = sigmoidf_(zv), n = load_as_f32(y, base + j, dt) * r;
            const float dn = go * w[j] * zv * s;
            store_from_f32(dy, base + j, r * (dn - n * mean), dt);
            store_from_f32(dz, base + j, go * n * w[j] * s * (1.f + zv * (1.f - s)), z_dt);
            sdw[wv][j] += go * n * zv * s;  // column j belongs to this lane within its wavefront
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < D; j += NT) {
        float s = 0.f;
        for (int g = 0; g < NT / 64; ++g) s += sdw[g][j];
        part[(size_t)blockIdx.x * D + j] = s;
    }
}

}  // namespace ops

// ------------------------------------------------------------------------------------------------ launchers

static unsigned nblocks(size_t n, size_t per) { return (unsigned)((n + per - 1) / per); }

static void launch_colsum(const float *part, int nrows, int ncols, float *out, float *out2, int split,
                          hipStream_t st) {
    if (ncols <= 0) return;
    if (nrows <= 128)
        hipLaunchKernelGGL(ops::colsum_thread_kernel, dim3(nblocks(ncols, ops::NT)), dim3(ops::NT), 0, st, part, nrows,
                           ncols, out, out2, split);
    else
        hipLaunchKernelGGL(ops::colsum_block_kernel, dim3(ncols), dim3(ops::NT), 0, st, part, nrows, ncols, out, out2,
                           split);
}

// Lanes per row for the vector row kernels: D = 8L with L a power of two in [4, 64]; 0 = generic path.
int row_lanes(int D) {
    if (D % 8) return 0;
    const int L = D / 8;
    return (L >= 4 && L <= 64 && (L & (L - 1)) == 0) ? L : 0;
}

void launch_gates_fwd(const void *a, const void *b, const float *A_log, const float *dt_bias, float *g, float *beta,
                      size_t tokens, int Hv, int in_dt, int log_space, float beta_scale, hipStream_t st) {
    const size_t n = tokens * Hv;
    if (n)
        hipLaunchKernelGGL(ops::gates_fwd_kernel, dim3(nblocks(n, ops::NT)), dim3(ops::NT), 0, st, a, b, A_log, dt_bias,
                           g, beta, n, Hv, in_dt, log_space, beta_scale);
}

int gates_max_heads() { return ops::NT; }

size_t gates_bwd_work_floats(size_t tokens, int Hv) { return (size_t)nblocks(tokens, ops::GATE_TOK) * Hv * 2; }

void launch_gates_bwd(const void *a, const void *b, const float *A_log, const float *dt_bias, const float *g,
                      const float *dg, const float *dbeta, void *da, void *db, float *dA_log, float *ddt_bias,
                      float *work, size_t tokens, int Hv, int in_dt, int grad_dt, int log_space, float beta_scale,
                      hipStream_t st) {
    const unsigned nblk = nblocks(tokens, ops::GATE_TOK);
    if (nblk)
        hipLaunchKernelGGL(ops::gates_bwd_kernel, dim3(nblk), dim3(ops::NT), 0, st, a, b, A_log, dt_bias, g, dg, dbeta,
                           da, db, work, tokens, Hv, in_dt, grad_dt, log_space, beta_scale);
    launch_colsum(work, (int)nblk, 2 * Hv, dA_log, ddt_bias, Hv, st);  // partial rows are [dA_log | ddt_bias]
}

void launch_l2norm_fwd(const void *x, void *y, size_t rows, int D, float eps, float scale, int dt, bool vec,
                       hipStream_t st) {
    if (!rows) return;
    const int L = vec ? row_lanes(D) : 0;
    switch (L) {
#define GDN_L2F(LL)                                                                                                   \
    case LL:                                                                                                          \
        hipLaunchKernelGGL(ops::l2norm_fwd_vec<LL>, dim3(nblocks(rows, ops::NT / LL)), dim3(ops::NT), 0, st, x, y,   \
                           rows, eps, scale, dt);                                                                     \
        break;
        GDN_L2F(4) GDN_L2F(8) GDN_L2F(16) GDN_L2F(32) GDN_L2F(64)
#undef GDN_L2F
    default:
        hipLaunchKernelGGL(ops::l2norm_fwd_any, dim3(nblocks(rows, ops::NT / 64)), dim3(ops::NT), 0, st, x, y, rows,
                           D, eps, scale, dt);
    }
}

void launch_l2norm_bwd(const void *x, const void *dy, void *dx, size_t rows, int D, float eps, float scale, int dt,
                       int dy_dt, bool vec, hipStream_t st) {
    if (!rows) return;
    const int L = vec ? row_lanes(D) : 0;
    switch (L) {
#define GDN_L2B(LL)                                                                                                   \
    case LL:                                                                                                          \
        hipLaunchKernelGGL(ops::l2norm_bwd_vec<LL>, dim3(nblocks(rows, ops::NT / LL)), dim3(ops::NT), 0, st, x, dy,  \
                           dx, rows, eps, scale, dt, dy_dt);                                                          \
        break;
        GDN_L2B(4) GDN_L2B(8) GDN_L2B(16) GDN_L2B(32) GDN_L2B(64)
#undef GDN_L2B
    default:
        hipLaunchKernelGGL(ops::l2norm_bwd_any, dim3(nblocks(rows, ops::NT / 64)), dim3(ops::NT), 0, st, x, dy, dx,
                           rows, D, eps, scale, dt, dy_dt);
    }
}

int conv_kmax() { return 8; }

static dim3 conv_grid(int B, int T, int C, int V) {
    return dim3(nblocks(C, 64 * V), nblocks(T, ops::CONV_SLICES * ops::CONV_TT), B);
}

// Channels per lane: 8 when x and q/k/v are 16-bit (16-byte loads), 4 when either is fp32 (or C % 8 != 0),
// 1 without aligned buffers; the backward holds a K-token window per channel, so it takes at most 4.
static int conv_lanes(int C, int dt, int g_dt, bool vec, bool bwd) {
    if (!vec || C % 4) return 1;
    const bool half = dt != DT_F32 && g_dt != DT_F32;
    return (half && C % 8 == 0 && !bwd) ? 8 : 4;
}

template <int K, int V, int L, int DT>
static void conv_launch_dt(const ops::ConvArgs &a, int B, bool bwd, hipStream_t st) {
    const dim3 grid = conv_grid(B, a.T, a.C, V);
    if (!bwd)
        hipLaunchKernelGGL((ops::conv_fwd_kernel<K, V, 4, L, DT>), grid, dim3(ops::NT), 0, st, a);
    else if constexpr (V <= 4)  // conv_lanes never gives the backward 8 channels per lane
        hipLaunchKernelGGL((ops::conv_bwd_kernel<K, V, 4, L, DT>), grid, dim3(ops::NT), 0, st, a);
}

// The vector paths with one dtype throughout (bf16 or fp32) run kernels with that dtype fixed at compile time.
template <int K, int V, int L>
static void conv_launch(const ops::ConvArgs &a, int B, bool bwd, hipStream_t st) {
    if constexpr (V >= 4) {
        if (a.dt == a.g_dt && a.dt == DT_BF16) return conv_launch_dt<K, V, L, DT_BF16>(a, B, bwd, st);
        if (a.dt == a.g_dt && a.dt == DT_F32) return conv_launch_dt<K, V, L, DT_F32>(a, B, bwd, st);
    }
    conv_launch_dt<K, V, L, -1>(a, B, bwd, st);
}

template <int K>
static void conv_plain(const ops::ConvArgs &a, int B, int V, bool bwd, hipStream_t st) {
    if (V == 8)
        conv_launch<K, 8, 0>(a, B, bwd, st);
    else if (V == 4)
        conv_launch<K, 4, 0>(a, B, bwd, st);
    else
        conv_launch<K, 1, 0>(a, B, bwd, st);
}

// Lanes per q/k head of the fused kernels (a power of two in [4, 64]) for V channels per lane, or 0.
static int conv_head_lanes(int Dk, int V) {
    if (Dk % V) return 0;
    const int L = Dk / V;
    return (L >= 4 && L <= 64 && (L & (L - 1)) == 0) ? L : 0;
}

bool conv_qkv_supported(int Dk, int K, int dt, int g_dt, bool vec, int C) {
    if (K != 4) return false;
    const int Vf = conv_lanes(C, dt, g_dt, vec, false), Vb = conv_lanes(C, dt, g_dt, vec, true);
    return Vf > 1 && Vb > 1 && conv_head_lanes(Dk, Vf) && conv_head_lanes(Dk, Vb);
}

// Dispatch: a.qk == 0 is the plain conv (any K in [2, 8]); a.qk > 0 the fused split + L2 norm (K = 4, checked by
// the caller with conv_qkv_supported).
static void conv_dispatch(const ops::ConvArgs &a, int B, int K, int Dk, bool vec, bool bwd, hipStream_t st) {
    const int V = conv_lanes(a.C, a.dt, a.g_dt, vec, bwd);
    if (a.qk > 0) {
        switch (conv_head_lanes(Dk, V) * 16 + V) {
        case 4 * 16 + 4: conv_launch<4, 4, 4>(a, B, bwd, st); break;
        case 8 * 16 + 4: conv_launch<4, 4, 8>(a, B, bwd, st); break;
        case 16 * 16 + 4: conv_launch<4, 4, 16>(a, B, bwd, st); break;
        case 32 * 16 + 4: conv_launch<4, 4, 32>(a, B, bwd, st); break;
        case 64 * 16 + 4: conv_launch<4, 4, 64>(a, B, bwd, st); break;
        case 4 * 16 + 8: conv_launch<4, 8, 4>(a, B, bwd, st); break;
        case 8 * 16 + 8: conv_launch<4, 8, 8>(a, B, bwd, st); break;
        case 16 * 16 + 8: conv_launch<4, 8, 16>(a, B, bwd, st); break;
        case 32 * 16 + 8: conv_launch<4, 8, 32>(a, B, bwd, st); break;
        case 64 * 16 + 8: conv_launch<4, 8, 64>(a, B, bwd, st); break;
        default: break;
        }
        return;
    }
    switch (K) {
    case 2: conv_plain<2>(a, B, V, bwd, st); break;
    case 3: conv_plain<3>(a, B, V, bwd, st); break;
    case 4: conv_plain<4>(a, B, V, bwd, st); break;
    case 5: conv_plain<5>(a, B, V, bwd, st); break;
    case 6: conv_plain<6>(a, B, V, bwd, st); break;
    case 7: conv_plain<7>(a, B, V, bwd, st); break;
    case 8: conv_plain<8>(a, B, V, bwd, st); break;
    default: break;
    }
}

void launch_conv_fwd(const ConvCall &c, hipStream_t st) {
    if (c.B && c.T && c.C) {
        ops::ConvArgs a{};
        a.x = c.x; a.w = c.w; a.state_in = c.state_in;
        a.q = c.q; a.k = c.k; a.v = c.v;
        a.T = c.T; a.C = c.C; a.qk = c.qk; a.dt = c.dt; a.g_dt = c.dt;
        a.scale_q = c.scale_q; a.eps = c.eps;
        conv_dispatch(a, c.B, c.K, c.Dk, c.vec, false, st);
    }
    if (c.state_out && c.B && c.C)
        hipLaunchKernelGGL(ops::conv_state_kernel, dim3(nblocks((size_t)c.B * (c.K - 1) * c.C, ops::NT)),
                           dim3(ops::NT), 0, st, c.x, c.state_in, c.state_out, c.B, c.T, c.C, c.K, c.dt);
}

size_t conv_bwd_work_floats(int B, int T, int C, int K) {
    return (size_t)B * nblocks(T, ops::CONV_SLICES * ops::CONV_TT) * C * K;
}

void launch_conv_bwd(const ConvCall &c, hipStream_t st) {
    if (!c.C) return;
    const int nparts = (c.B && c.T) ? (int)(c.B * nblocks(c.T, ops::CONV_SLICES * ops::CONV_TT)) : 0;
    if (nparts) {
        ops::ConvArgs a{};
        a.x = c.x; a.w = c.w; a.state_in = c.state_in;
        a.q = c.q; a.k = c.k; a.v = c.v; a.dx = c.dx; a.part = c.work;
        a.T = c.T; a.C = c.C; a.qk = c.qk; a.dt = c.dt; a.g_dt = c.g_dt;
        a.scale_q = c.scale_q; a.eps = c.eps;
        conv_dispatch(a, c.B, c.K, c.Dk, c.vec, true, st);
    }
    launch_colsum(c.work, nparts, c.C * c.K, c.dw, c.dw, c.C * c.K, st);  // with no tokens: dw = 0
}

int grms_dmax() { return ops::GRMS_DMAX; }

void launch_grms_fwd(const void *y, const void *z, const float *w, void *out, size_t rows, int D, float eps, int dt,
                     int z_dt, bool vec, hipStream_t st) {
    if (!rows) return;
    const int L = vec ? row_lanes(D) : 0;
    switch (L) {
#define GDN_GF(LL)                                                                                                    \
    case LL:                                                                                                          \
        hipLaunchKernelGGL(ops::grms_fwd_vec<LL>, dim3(nblocks(rows, ops::NT / LL)), dim3(ops::NT), 0, st, y, z, w,  \
                           out, rows, eps, dt, z_dt);                                                                 \
        break;
        GDN_GF(4) GDN_GF(8) GDN_GF(16) GDN_GF(32) GDN_GF(64)
#undef GDN_GF
    default:
        hipLaunchKernelGGL(ops::grms_fwd_any, dim3(nblocks(rows, ops::NT / 64)), dim3(ops::NT), 0, st, y, z, w, out,
                           rows, D, eps, dt, z_dt);
    }
}

size_t grms_bwd_work_floats(size_t rows, int D) { return (size_t)nblocks(rows, ops::GRMS_ROWS) * D; }

void launch_grms_bwd(const void *y, const void *z, const float *w, const void *dout, void *dy, void *dz, float *dw,
                     float *work, size_t rows, int D, float eps, int dt, int z_dt, int dout_dt, bool vec,
                     hipStream_t st) {
    const unsigned nblk = nblocks(rows, ops::GRMS_ROWS);
    const int L = vec ? row_lanes(D) : 0;
    if (nblk) {
        switch (L) {
#define GDN_GB(LL)                                                                                                    \
    case LL:                                                                                                          \
        hipLaunchKernelGGL(ops::grms_bwd_vec<LL>, dim3(nblk), dim3(ops::NT), 0, st, y, z, w, dout, dy, dz, work,     \
                           rows, eps, dt, z_dt, dout_dt);                                                             \
        break;
            GDN_GB(4) GDN_GB(8) GDN_GB(16) GDN_GB(32) GDN_GB(64)
#undef GDN_GB
        default:
            hipLaunchKernelGGL(ops::grms_bwd_any, dim3(nblk), dim3(ops::NT), 0, st, y, z, w, dout, dy, dz, work, rows,
                               D, eps, dt, z_dt, dout_dt);
        }
    }
    launch_colsum(work, (int)nblk, D, dw, dw, D, st);  // with no rows: dw = 0
}

}  // namespace gdn
