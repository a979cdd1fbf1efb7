// Masked steps on the chunked form: the elementwise pieces around two chunked passes.
//
// A step with mask m_t = 0 keeps the state (S_t = S_{t-1}) but its output reads the candidate state
// (tools/gdn_vjp.py:3-6, _step_parts :238-256):
//   y_t = S~_t q_t = d_t S_{t-1} q_t + beta_t (k_t . q_t) (v_t - d_t S_{t-1} k_t)          (d_t the decay).
// The chunked form runs the effective recurrence with d'_t = m_t ? d_t : 1 and beta'_t = m_t beta_t, whose state
// equals the masked recurrence's state at every token.  Its output y'_t = S'_t q_t is y_t where m_t = 1 and
// S_{t-1} q_t where m_t = 0; a second pass with k as the query gives z_t = S'_t k_t = S_{t-1} k_t there.  Then at
// masked tokens, with c = k_t . q_t (the value head's key head) and u = v_t - d_t z_t:
//   y_t = d_t y'_t + beta_t c u
// and the VJP of that expression feeds the two passes' backwards:
//   dy'_t = d_t dy_t,  dz_t = -beta_t c d_t dy_t,  dv_t += beta_t c dy_t,  dbeta_t = c (u . dy_t),
//   dd_t = (y'_t - beta_t c z_t) . dy_t,  dq_t += beta_t (u . dy_t) k_t,  dk_t += beta_t (u . dy_t) q_t
// (dq / dk summed over the value heads of a key head).  Unmasked tokens pass dy through to the first pass.
#include "gdn_common.h"
#include "gdn_internal.h"

namespace gdn {

constexpr int MK_THREADS = 256;
constexpr int MK_MAX_HEADS = 256;

__global__ __launch_bounds__(256) void mask_gates_kernel(const float *g, const float *beta, const uint8_t *mask,
                                                         float *g2, float *beta2, size_t n, int Hv, int gate) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const bool keep = mask[i / Hv] != 0;
    g2[i] = keep ? g[i] : (gate == GATE_LOG ? 0.f : 1.f);
    beta2[i] = keep ? beta[i] : 0.f;
}

// Sum over the wave, the same bits in every lane: DPP row sums, then the lane swaps across rows and halves.
__device__ __forceinline__ float wave_sum(float x) {
    x = row16_allreduce(x);
    x += lane_xor16(x);
    return x + lane_xor32(x);
}

// Four consecutive elements (i % 4 == 0) of a tensor of dtype dt, as fp32 / from fp32.
__device__ __forceinline__ float4 load4(const void *p, size_t i, int dt) {
    if (dt == DT_F32) return *reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
    if (dt == DT_BF16) {
        const uint2 w = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(p) + i);
        return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                           __uint_as_float(w.y & 0xffff0000u));
    }
    return make_float4(load_as_f32(p, i, dt), load_as_f32(p, i + 1, dt), load_as_f32(p, i + 2, dt),
                       load_as_f32(p, i + 3, dt));
}
__device__ __forceinline__ void store4(void *p, size_t i, float4 x, int dt) {
    if (dt == DT_F32) {
        *reinterpret_cast<float4 *>(static_cast<float *>(p) + i) = x;
    } else if (dt == DT_BF16) {
        const uint32_t a = f32_to_bf16_cvt(x.x) | ((uint32_t)f32_to_bf16_cvt(x.y) << 16);
        const uint32_t b = f32_to_bf16_cvt(x.z) | ((uint32_t)f32_to_bf16_cvt(x.w) << 16);
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p) + i) = make_uint2(a, b);
    } else {
        store_from_f32(p, i, x.x, dt);
        store_from_f32(p, i + 1, x.y, dt);
        store_from_f32(p, i + 2, x.z, dt);
        store_from_f32(p, i + 3, x.w, dt);
    }
}
__device__ __forceinline__ float4 ld4f(const float *p, size_t i) { return *reinterpret_cast<const float4 *>(p + i); }
__device__ __forceinline__ float4 add4(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }
__device__ __forceinline__ float4 fma4(float s, float4 a, float4 b) {
    return make_float4(fmaf(s, a.x, b.x), fmaf(s, a.y, b.y), fmaf(s, a.z, b.z), fmaf(s, a.w, b.w));
}

__device__ __forceinline__ float decay_of(const float *g, size_t gi, int gate) {
    return gate == GATE_LOG ? expf(g[gi]) : g[gi];
}

// c[hk] = k_t . q_t for every key head of token tok, one wave per key head (ends with a barrier).
__device__ __forceinline__ void key_dots(const MaskArgs &a, size_t tok, float *c) {
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    for (int hk = w; hk < a.Hk; hk += MK_THREADS / 64) {
        const size_t base = (tok * a.Hk + hk) * a.Dk;
        float s = 0.f;
        for (int j = l; j < a.Dk; j += 64) s += load_as_f32(a.q, base + j, a.in_dt) * load_as_f32(a.k, base + j, a.in_dt);
        s = wave_sum(s);
        if (l == 0) c[hk] = s;
    }
    __syncthreads();
}

// Forward fix-up: y <- d y' + beta c (v - d z) at masked tokens, y' elsewhere.  With Yp set, y' is the first pass's
// fp32 output there (kept for the backward) and every token's y is written; without, y holds y' in its own dtype
// and only masked tokens are rewritten.
__global__ __launch_bounds__(MK_THREADS) void mask_fix_fwd_kernel(MaskArgs a) {
    const size_t tok = blockIdx.x;
    const bool keep = a.mask[tok] != 0;
    if (keep && !a.Yp) return;
    __shared__ float c[MK_MAX_HEADS];
    if (!keep) key_dots(a, tok, c);
    const int rep = a.Hv / a.Hk;
    // four consecutive elements per thread and step (Dv % 4 == 0)
    for (int e = 4 * threadIdx.x; e < a.Hv * a.Dv; e += 4 * MK_THREADS) {
        const size_t vi = tok * a.Hv * a.Dv + e;
        float4 y = a.Yp ? ld4f(a.Yp, vi) : load4(a.y, vi, a.out_dt);
        if (!keep) {
            const int hv = e / a.Dv;
            const size_t gi = tok * a.Hv + hv;
            const float d = decay_of(a.g, gi, a.gate), bc = a.beta[gi] * c[hv / rep];
            const float4 v = load4(a.v, vi, a.in_dt), z = ld4f(a.Z, vi);
            y = make_float4(d * y.x + bc * (v.x - d * z.x), d * y.y + bc * (v.y - d * z.y), d * y.z + bc * (v.z - d * z.z),
                            d * y.w + bc * (v.w - d * z.w));
        }
        store4(a.y, vi, y, a.out_dt);
    }
}

// Cotangents of the two passes: dy1 = (masked ? d dy : dy), dz = (masked ? -beta c d dy : 0), both fp32; four
// consecutive elements per thread and step (Dv % 4 == 0).
__global__ __launch_bounds__(MK_THREADS) void mask_bwd_cot_kernel(MaskArgs a) {
    const size_t tok = blockIdx.x;
    const bool keep = a.mask[tok] != 0;
    __shared__ float c[MK_MAX_HEADS];
    if (!keep) key_dots(a, tok, c);
    const int rep = a.Hv / a.Hk;
    for (int e = 4 * threadIdx.x; e < a.Hv * a.Dv; e += 4 * MK_THREADS) {
        const size_t vi = tok * a.Hv * a.Dv + e;
        const float4 dy = load4(a.dy, vi, a.dy_dt);
        float s1 = 1.f, sz = 0.f;
        if (!keep) {
            const int hv = e / a.Dv;
            const size_t gi = tok * a.Hv + hv;
            s1 = decay_of(a.g, gi, a.gate);
            sz = -a.beta[gi] * c[hv / rep] * s1;
        }
        *reinterpret_cast<float4 *>(a.dy1 + vi) = make_float4(s1 * dy.x, s1 * dy.y, s1 * dy.z, s1 * dy.w);
        *reinterpret_cast<float4 *>(a.dz + vi) = make_float4(sz * dy.x, sz * dy.y, sz * dy.z, sz * dy.w);
    }
}

// Gradients: the two passes' fp32 parts summed (pass 2 ran with k as its query, so its dq adds to dk), the
// chunked gate gradients kept where m = 1, and the fix-up's terms added where m = 0.
__global__ __launch_bounds__(MK_THREADS) void mask_bwd_combine_kernel(MaskArgs a) {
    const size_t tok = blockIdx.x;
    const bool keep = a.mask[tok] != 0;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, rep = a.Hv / a.Hk;
    __shared__ float c[MK_MAX_HEADS], su[MK_MAX_HEADS], sd[MK_MAX_HEADS];
    if (!keep) {
        key_dots(a, tok, c);
        for (int hv = w; hv < a.Hv; hv += MK_THREADS / 64) {
            const size_t gi = tok * a.Hv + hv, base = gi * a.Dv;
            const float d = decay_of(a.g, gi, a.gate), bc = a.beta[gi] * c[hv / rep];
            float s = 0.f, dd = 0.f;
            for (int i = l; i < a.Dv; i += 64) {
                const float dy = load_as_f32(a.dy, base + i, a.dy_dt), z = a.Z[base + i];
                s += (load_as_f32(a.v, base + i, a.in_dt) - d * z) * dy;
                dd += (a.Yp[base + i] - bc * z) * dy;
            }
            s = wave_sum(s);
            dd = wave_sum(dd);
            if (l == 0) {
                su[hv] = s;
                sd[hv] = dd;
            }
        }
        __syncthreads();
    }
    // four consecutive elements per thread and step (Dk, Dv % 4 == 0)
    for (int e = 4 * tid; e < a.Hk * a.Dk; e += 4 * MK_THREADS) {
        const int hk = e / a.Dk;
        const size_t i = tok * a.Hk * a.Dk + e;
        float4 dq = ld4f(a.dq1, i), dk = add4(add4(ld4f(a.dk1, i), ld4f(a.dk2, i)), ld4f(a.dq2, i));
        if (!keep) {
            float f = 0.f;
            for (int r = 0; r < rep; ++r) {
                const int hv = hk * rep + r;
                f += a.beta[tok * a.Hv + hv] * su[hv];
            }
            dq = fma4(f, load4(a.k, i, a.in_dt), dq);
            dk = fma4(f, load4(a.q, i, a.in_dt), dk);
        }
        store4(a.dq, i, dq, a.grad_dt);
        store4(a.dk, i, dk, a.grad_dt);
    }
    for (int e = 4 * tid; e < a.Hv * a.Dv; e += 4 * MK_THREADS) {
        const size_t i = tok * a.Hv * a.Dv + e;
        float4 dv = add4(ld4f(a.dv1, i), ld4f(a.dv2, i));
        if (!keep) {
            const int hv = e / a.Dv;
            dv = fma4(a.beta[tok * a.Hv + hv] * c[hv / rep], load4(a.dy, i, a.dy_dt), dv);
        }
        store4(a.dv, i, dv, a.grad_dt);
    }
    for (int hv = tid; hv < a.Hv; hv += MK_THREADS) {
        const size_t gi = tok * a.Hv + hv;
        if (keep) {
            a.dg[gi] = a.dg1[gi] + a.dg2[gi];
            a.dbeta[gi] = a.dbeta1[gi] + a.dbeta2[gi];
        } else {
            a.dg[gi] = a.gate == GATE_LOG ? decay_of(a.g, gi, a.gate) * sd[hv] : sd[hv];
            a.dbeta[gi] = c[hv / rep] * su[hv];
        }
    }
}

__global__ __launch_bounds__(256) void add2_kernel(float *dst, const float *x, const float *y, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = x[i] + y[i];
}

int mask_max_heads() { return MK_MAX_HEADS; }

void launch_mask_gates(const float *g, const float *beta, const uint8_t *mask, float *g2, float *beta2,
                       size_t tokens, int Hv, int gate, hipStream_t st) {
    const size_t n = tokens * Hv;
    if (n) hipLaunchKernelGGL(mask_gates_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, beta, mask,
                              g2, beta2, n, Hv, gate);
}

void launch_mask_fix_fwd(const MaskArgs &a, size_t tokens, hipStream_t st) {
    if (tokens) hipLaunchKernelGGL(mask_fix_fwd_kernel, dim3((unsigned)tokens), dim3(MK_THREADS), 0, st, a);
}

void launch_mask_bwd_cot(const MaskArgs &a, size_t tokens, hipStream_t st) {
    if (tokens) hipLaunchKernelGGL(mask_bwd_cot_kernel, dim3((unsigned)tokens), dim3(MK_THREADS), 0, st, a);
}

void launch_mask_bwd_combine(const MaskArgs &a, size_t tokens, hipStream_t st) {
    if (tokens) hipLaunchKernelGGL(mask_bwd_combine_kernel, dim3((unsigned)tokens), dim3(MK_THREADS), 0, st, a);
}

void launch_add2(float *dst, const float *x, const float *y, size_t n, hipStream_t st) {
    if (dst && n) hipLaunchKernelGGL(add2_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dst, x, y, n);
}

}  // namespace gdn
