// Shared device/host helpers for the STAR-KV paged decode library (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/starkv_hip.h"

namespace starkv {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Error reporting through the C ABI: a thread-local message, nonzero return.
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

#define SKV_CHECK(cond, ...)                 \
    do {                                      \
        if (!(cond)) {                        \
            ::starkv::set_error(__VA_ARGS__); \
            return STARKV_ERR_ARG;            \
        }                                     \
    } while (0)

#define SKV_HIP(call)                                                            \
    do {                                                                         \
        hipError_t e_ = (call);                                                  \
        if (e_ != hipSuccess) {                                                  \
            ::starkv::set_error("%s failed: %s", #call, hipGetErrorString(e_)); \
            return STARKV_ERR_HIP;                                               \
        }                                                                        \
    } while (0)

// ---------------------------------------------------------------------------
// Scalar conversions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float load_f(const void* p, int64_t i, int dt) {
    if (dt == STARKV_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    if (dt == STARKV_F16) return (float)((const _Float16*)p)[i];
    return ((const float*)p)[i];
}

__device__ __forceinline__ void store_f(void* p, int64_t i, int dt, float v) {
    if (dt == STARKV_BF16)
        ((uint16_t*)p)[i] = f32_to_bf16_rne(v);
    else if (dt == STARKV_F16)
        ((_Float16*)p)[i] = (_Float16)v;
    else
        ((float*)p)[i] = v;
}

// Eight consecutive elements starting at element i (16-byte aligned for 2-byte
// types, 32-byte for fp32) as fp32.
__device__ __forceinline__ void load8_f(const void* p, int64_t i, int dt, float* o) {
    if (dt == STARKV_F32) {
        const float4* v = (const float4*)((const float*)p + i);
        float4 a = v[0], b = v[1];
        o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
        o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
        return;
    }
    uint4 w = *(const uint4*)((const uint16_t*)p + i);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    if (dt == STARKV_BF16) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o[2 * k] = __uint_as_float(ws[k] << 16);
            o[2 * k + 1] = __uint_as_float(ws[k] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            _Float16 lo, hi;
            uint16_t l16 = (uint16_t)(ws[k] & 0xffffu), h16 = (uint16_t)(ws[k] >> 16);
            memcpy(&lo, &l16, 2);
            memcpy(&hi, &h16, 2);
            o[2 * k] = (float)lo;
            o[2 * k + 1] = (float)hi;
        }
    }
}

__device__ __forceinline__ int dtype_size(int dt) { return dt == STARKV_F32 ? 4 : 2; }

// A value the optimizer cannot see through: address arithmetic derived from it is
// recomputed where it is used instead of being hoisted out of the main loop and
// held in registers for the whole kernel.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// The same for a wave-uniform value (kept in an SGPR): comparisons and products of it
// are redone where used rather than hoisted into SGPRs that live across the loop.
__device__ __forceinline__ int opaque_s(int v) {
    asm volatile("" : "+s"(v));
    return v;
}

// A per-lane value pinned whole in one VGPR: a lane address computed once stays one
// register, instead of being split into a wave-uniform SGPR part and a VGPR part that
// every use adds back together.
__device__ __forceinline__ uint32_t vgpr_pin(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}


// Reductions over the 16 lanes of a row (lanes 16r .. 16r+15) with DPP: quad_perm
// [1,0,3,2] (0xB1), quad_perm [2,3,0,1] (0x4E), row_half_mirror (0x141), row_mirror
// (0x140). Every source lane lies inside the row, so no lane reads a disabled one.
template <int CTL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTL, 0xF, 0xF, true));
}

__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}

__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return v;
}

// Sums over the 4 rows of a wave (lanes l, l^16, l^32, l^48) with the gfx950 lane
// swaps. v_permlane32_swap(a, b) leaves a = {a[0:32), b[0:32)}, b = {a[32:64), b[32:64)};
// v_permlane16_swap(a, b) leaves a = {a.R0, b.R0, a.R2, b.R2}, b = {a.R1, b.R1, a.R3, b.R3}
// (Rk = lanes 16k .. 16k+15).
__device__ __forceinline__ float sum_rows(float v) {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(x[0]) + __uint_as_float(x[1]);
    const auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(y[0]) + __uint_as_float(y[1]);
}

// Four row sums at once. The result's row 0 holds the sum of a, row 1 of c, row 2 of b,
// row 3 of d (each over the 4 rows of its input).
__device__ __forceinline__ float sum_rows4(float a, float b, float c, float d) {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    const float X = __uint_as_float(x[0]) + __uint_as_float(x[1]);  // {a02, a13, b02, b13}
    const auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(d), false, false);
    const float Y = __uint_as_float(y[0]) + __uint_as_float(y[1]);  // {c02, c13, d02, d13}
    const auto z = __builtin_amdgcn_permlane16_swap(__float_as_uint(X), __float_as_uint(Y), false, false);
    return __uint_as_float(z[0]) + __uint_as_float(z[1]);           // {a, c, b, d}
}

// Max over the 4 rows of a wave (lanes l, l^16, l^32, l^48), as sum_rows.
__device__ __forceinline__ float max_rows(float v) {
    const auto x = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
    const auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return fmaxf(__uint_as_float(y[0]), __uint_as_float(y[1]));
}

// Wave64 reductions (every lane active, every lane gets the result): within each row of
// 16 with DPP, then over the rows with the lane swaps.
__device__ __forceinline__ float wave_max(float v) { return max_rows(row16_max(v)); }
__device__ __forceinline__ float wave_sum(float v) { return sum_rows(row16_sum(v)); }

// ---------------------------------------------------------------------------
// s_waitcnt with a run-time count (the instruction takes an immediate).
// gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in 15:14, expcnt 6:4,
// lgkmcnt 11:8.
// ---------------------------------------------------------------------------
#define SKV_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (0 << 8))

__device__ __forceinline__ void wait_vmcnt_lgkm0(int n) {
    switch (n) {
        case 0: SKV_WAIT_VM_LGKM0(0); break;
        case 1: SKV_WAIT_VM_LGKM0(1); break;
        case 2: SKV_WAIT_VM_LGKM0(2); break;
        case 3: SKV_WAIT_VM_LGKM0(3); break;
        case 4: SKV_WAIT_VM_LGKM0(4); break;
        case 5: SKV_WAIT_VM_LGKM0(5); break;
        case 6: SKV_WAIT_VM_LGKM0(6); break;
        case 7: SKV_WAIT_VM_LGKM0(7); break;
        case 8: SKV_WAIT_VM_LGKM0(8); break;
        case 9: SKV_WAIT_VM_LGKM0(9); break;
        case 10: SKV_WAIT_VM_LGKM0(10); break;
        case 11: SKV_WAIT_VM_LGKM0(11); break;
        case 12: SKV_WAIT_VM_LGKM0(12); break;
        case 13: SKV_WAIT_VM_LGKM0(13); break;
        case 14: SKV_WAIT_VM_LGKM0(14); break;
        case 15: SKV_WAIT_VM_LGKM0(15); break;
        default: SKV_WAIT_VM_LGKM0(0); break;
    }
}

// The same for counts up to 63 (rounded down to a multiple of 4 above 15, which only
// waits for more).
__device__ __forceinline__ void wait_vmcnt_lgkm0_wide(int n) {
    if (n <= 15) {
        wait_vmcnt_lgkm0(n);
        return;
    }
    switch (min(n, 63) >> 2) {
        case 4: SKV_WAIT_VM_LGKM0(16); break;
        case 5: SKV_WAIT_VM_LGKM0(20); break;
        case 6: SKV_WAIT_VM_LGKM0(24); break;
        case 7: SKV_WAIT_VM_LGKM0(28); break;
        case 8: SKV_WAIT_VM_LGKM0(32); break;
        case 9: SKV_WAIT_VM_LGKM0(36); break;
        case 10: SKV_WAIT_VM_LGKM0(40); break;
        case 11: SKV_WAIT_VM_LGKM0(44); break;
        case 12: SKV_WAIT_VM_LGKM0(48); break;
        case 13: SKV_WAIT_VM_LGKM0(52); break;
        case 14: SKV_WAIT_VM_LGKM0(56); break;
        default: SKV_WAIT_VM_LGKM0(60); break;
    }
}

// Workgroup barrier that does not drain outstanding global->LDS copies: the
// caller has already waited for what it needs (lgkmcnt(0) included). The empty asm
// keeps the compiler from moving LDS accesses across it (the barrier intrinsic itself
// is not a memory operation to the optimizer).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ void wait_lgkm0_barrier() {
    __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0) only
    __builtin_amdgcn_s_barrier();
}

}  // namespace starkv
