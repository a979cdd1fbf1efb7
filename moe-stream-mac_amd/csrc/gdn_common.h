// Device helpers shared by the GDN kernels: dtype conversion and wavefront reductions for gfx950.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace gdn {

enum : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
enum : int { GATE_DECAY = 0, GATE_DECAY_VEC = 1, GATE_LOG = 2, GATE_LOG_VEC = 3 };
// one gate value per key channel ([B][T][Hv][Dk]) rather than per head; the gate given as the log decay
__host__ __device__ constexpr bool gate_vec(int gate) { return gate == GATE_DECAY_VEC || gate == GATE_LOG_VEC; }
__host__ __device__ constexpr bool gate_in_log(int gate) { return gate == GATE_LOG || gate == GATE_LOG_VEC; }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even float -> bfloat16 (NaN stays a quiet NaN), in integer arithmetic.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
// The same rounding by gfx950's v_cvt_pk_bf16_f32 (no branch): faster for scattered single-element stores.
__device__ __forceinline__ uint16_t f32_to_bf16_cvt(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Load element i of a buffer of dtype dt as float.  dt is uniform across the wave.
__device__ __forceinline__ float load_as_f32(const void *p, size_t i, int dt) {
    if (dt == DT_F32) return static_cast<const float *>(p)[i];
    if (dt == DT_BF16) return bf16_to_f32(static_cast<const uint16_t *>(p)[i]);
    return __half2float(static_cast<const __half *>(p)[i]);
}

__device__ __forceinline__ void store_from_f32(void *p, size_t i, float x, int dt) {
    if (dt == DT_F32) {
        static_cast<float *>(p)[i] = x;
    } else if (dt == DT_BF16) {
        static_cast<uint16_t *>(p)[i] = f32_to_bf16_cvt(x);
    } else {
        static_cast<__half *>(p)[i] = __float2half(x);
    }
}

// Four consecutive elements from element i (i a multiple of 4, the buffer 16-byte aligned): one 16-byte store in
// fp32, one 8-byte store of packed bf16, element stores in fp16.
__device__ __forceinline__ void store4_from_f32(void *p, size_t i, float4 x, int dt) {
    if (dt == DT_F32) {
        *reinterpret_cast<float4 *>(static_cast<float *>(p) + i) = x;
    } else if (dt == DT_BF16) {
        const uint32_t lo = f32_to_bf16_cvt(x.x) | ((uint32_t)f32_to_bf16_cvt(x.y) << 16);
        const uint32_t hi = f32_to_bf16_cvt(x.z) | ((uint32_t)f32_to_bf16_cvt(x.w) << 16);
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(p) + i) = make_uint2(lo, hi);
    } else {
        __half *h = static_cast<__half *>(p) + i;
        h[0] = __float2half(x.x); h[1] = __float2half(x.y); h[2] = __float2half(x.z); h[3] = __float2half(x.w);
    }
}

// DPP lane moves inside a row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_1032 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

// Sum over the 16 lanes of a DPP row; every lane of the row receives the same (bitwise) total.
__device__ __forceinline__ float row16_allreduce(float x) {
    x += dpp_mov<DPP_QUAD_1032>(x);
    x += dpp_mov<DPP_QUAD_2301>(x);
    x += dpp_mov<DPP_ROW_HALF_MIRROR>(x);
    x += dpp_mov<DPP_ROW_MIRROR>(x);
    return x;
}

// Inclusive prefix sum over the 64 lanes (all active): Hillis-Steele inside each row of 16 lanes (row_shr 1, 2, 4, 8,
// out-of-row sources read 0), then the row totals carried by row_bcast:15 (rows 1 and 3) and row_bcast:31 (rows 2
// and 3).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_masked(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_prefix_sum(float x) {
    x += dpp_mov<0x111>(x);  // row_shr:1
    x += dpp_mov<0x112>(x);  // row_shr:2
    x += dpp_mov<0x114>(x);  // row_shr:4
    x += dpp_mov<0x118>(x);  // row_shr:8
    x += dpp_masked<0x142, 0xA>(x);  // row_bcast:15
    x += dpp_masked<0x143, 0xC>(x);  // row_bcast:31
    return x;
}
// The same scan in fp64 (each DPP move carries the two halves of a lane's double).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_mov_f64(double x) {
    const long long v = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(v & 0xffffffffll), CTRL, ROW_MASK, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(v >> 32), CTRL, ROW_MASK, 0xF, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ double wave_prefix_sum(double x) {
    x += dpp_mov_f64<0x111>(x);
    x += dpp_mov_f64<0x112>(x);
    x += dpp_mov_f64<0x114>(x);
    x += dpp_mov_f64<0x118>(x);
    x += dpp_mov_f64<0x142, 0xA>(x);
    x += dpp_mov_f64<0x143, 0xC>(x);
    return x;
}
// Lane `lane`'s double, read into every lane (a scalar read, no LDS round trip).
__device__ __forceinline__ double readlane_f64(double x, int lane) {
    const long long v = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_readlane((int)(v & 0xffffffffll), lane);
    const int hi = __builtin_amdgcn_readlane((int)(v >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
// Lane i receives lane i - 1 of the wave (lane 0 receives 0): wave_shr:1.
__device__ __forceinline__ float wave_shr1(float x) { return dpp_mov<0x138>(x); }

// The value of lane l ^ 16 / l ^ 32 on gfx950's VALU lane swaps (no LDS round trip): permlane16_swap exchanges
// the odd rows of its first operand with the even rows of its second, permlane32_swap the upper half of the first
// with the lower half of the second; with both operands x, a lane's partner is in the half it did not keep.
__device__ __forceinline__ float lane_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Two sums over lane pairs l, l ^ 16 with one swap: lanes of even 16-lane rows get a + a(l ^ 16), lanes of odd
// rows b + b(l ^ 16).  The swap leaves each lane holding the two addends it needs (a even lane keeps its a and
// receives its partner's a; an odd lane keeps its b and receives its partner's b).
__device__ __forceinline__ float pair_sum16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The same over lane pairs l, l ^ 32: the lower half gets a + a(l ^ 32), the upper half b + b(l ^ 32).
__device__ __forceinline__ float pair_sum32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace gdn
