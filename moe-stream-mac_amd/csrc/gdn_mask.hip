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

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
    return x;
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
    for (int e = threadIdx.x; e < a.Hv * a.Dv; e += MK_THREADS) {
        const size_t vi = tok * a.Hv * a.Dv + e;
        const float yp = a.Yp ? a.Yp[vi] : load_as_f32(a.y, vi, a.out_dt);
        float y = yp;
        if (!keep) {
            const int hv = e / a.Dv;
            const size_t gi = tok * a.Hv + hv;
            const float d = decay_of(a.g, gi, a.gate), bt = a.beta[gi];
            y = d * yp + bt * c[hv / rep] * (load_as_f32(a.v, vi, a.in_dt) - d * a.Z[vi]);
        }
        store_from_f32(a.y, vi, y, a.out_dt);
    }
}

// Cotangents of the two passes: dy1 = (masked ? d dy : dy), dz = (masked ? -beta c d dy : 0), both fp32.
__global__ __launch_bounds__(MK_THREADS) void mask_bwd_cot_kernel(MaskArgs a) {
    const size_t tok = blockIdx.x;
    const bool keep = a.mask[tok] != 0;
    __shared__ float c[MK_MAX_HEADS];
    if (!keep) key_dots(a, tok, c);
    const int rep = a.Hv / a.Hk;
    for (int e = threadIdx.x; e < a.Hv * a.Dv; e += MK_THREADS) {
        const size_t vi = tok * a.Hv * a.Dv + e;
        const float dy = load_as_f32(a.dy, vi, a.dy_dt);
        if (keep) {
            a.dy1[vi] = dy;
            a.dz[vi] = 0.f;
        } else {
            const int hv = e / a.Dv;
            const size_t gi = tok * a.Hv + hv;
            const float d = decay_of(a.g, gi, a.gate);
            a.dy1[vi] = d * dy;
            a.dz[vi] = -a.beta[gi] * c[hv / rep] * d * dy;
        }
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
    for (int e = tid; e < a.Hk * a.Dk; e += MK_THREADS) {
        const int hk = e / a.Dk;
        const size_t i = tok * a.Hk * a.Dk + e;
        float dq = a.dq1[i], dk = a.dk1[i] + a.dk2[i] + a.dq2[i];
        if (!keep) {
            float f = 0.f;
            for (int r = 0; r < rep; ++r) {
                const int hv = hk * rep + r;
                f += a.beta[tok * a.Hv + hv] * su[hv];
            }
            dq += f * load_as_f32(a.k, i, a.in_dt);
            dk += f * load_as_f32(a.q, i, a.in_dt);
        }
        store_from_f32(a.dq, i, dq, a.grad_dt);
        store_from_f32(a.dk, i, dk, a.grad_dt);
    }
    for (int e = tid; e < a.Hv * a.Dv; e += MK_THREADS) {
        const size_t i = tok * a.Hv * a.Dv + e;
        float dv = a.dv1[i] + a.dv2[i];
        if (!keep) {
            const int hv = e / a.Dv;
            dv += a.beta[tok * a.Hv + hv] * c[hv / rep] * load_as_f32(a.dy, i, a.dy_dt);
        }
        store_from_f32(a.dv, i, dv, a.grad_dt);
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
