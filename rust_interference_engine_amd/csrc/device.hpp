// device.hpp — device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace rie {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));


// Weight-stream loads.  Plain loads: on gfx950 the nontemporal form measured
// about 35% slower for the decode GEMVs (RIE_WEIGHT_NT=1 selects it).
#ifndef RIE_WEIGHT_NT
#define RIE_WEIGHT_NT 0
#endif
template <class T>
__device__ __forceinline__ T wload(const T *p) {
#if RIE_WEIGHT_NT
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}
__device__ __forceinline__ u32x4 ld_w16(const void *p) { return wload((const u32x4 *)p); }
__device__ __forceinline__ f32x4 ld_w16f(const void *p) { return wload((const f32x4 *)p); }

__device__ __forceinline__ float h2f(uint32_t bits16) {
    _Float16 h;
    uint16_t b = (uint16_t)bits16;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// IEEE round-to-nearest-even f32→f16 (v_cvt_f16_f32 in the default rounding mode)
__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 h = (_Float16)f;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ float wave_sum(float v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v, int width) {
    for (int o = width >> 1; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 32 bytes starting at a 2-byte aligned address p, as 8 little-endian dwords:
// 9 dword loads from the dword-aligned address below p, realigned by v_alignbyte.
// Reads up to 4 bytes past p+32 (device weight blobs carry slack for it).
__device__ __forceinline__ void load32_a2(const uint8_t *p, uint32_t out[8]) {
    uintptr_t a = (uintptr_t)p;
    const uint32_t *q = (const uint32_t *)(a & ~(uintptr_t)3);
    uint32_t sh = (uint32_t)(a & 3);
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 9; i++) w[i] = wload(q + i);
#pragma unroll
    for (int i = 0; i < 8; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float gelu_tanh_f(float x) {
    const float k = 0.7978846f;
    return 0.5f * x * (1.0f + tanhf(k * x * (1.0f + 0.044715f * x * x)));
}

// ---- DPP lane exchange (VALU, no LDS) ----
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_QUAD_XOR1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_ROR4 = 0x124;   // row_ror:4 (16-lane rows)
constexpr int DPP_ROW_ROR8 = 0x128;   // row_ror:8
constexpr int DPP_HALF_MIRROR = 0x141;  // row_half_mirror (8-lane halves)

// Sum over aligned groups of W lanes (W = 1..32, a power of two); every lane of
// the group receives the sum.  Call with the whole wavefront active.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (W >= 2) v += dpp_f<DPP_QUAD_XOR1>(v);
    if constexpr (W >= 4) v += dpp_f<DPP_QUAD_XOR2>(v);
    if constexpr (W == 8) v += dpp_f<DPP_HALF_MIRROR>(v);
    if constexpr (W >= 16) {
        v += dpp_f<DPP_ROW_ROR4>(v);
        v += dpp_f<DPP_ROW_ROR8>(v);
    }
    if constexpr (W == 32) v += __shfl_xor(v, 16, 64);
    return v;
}
// exact integer sum over the 4 lanes of a quad
__device__ __forceinline__ int quad_sum_i(int v) {
    v += dpp_i<DPP_QUAD_XOR1>(v);
    v += dpp_i<DPP_QUAD_XOR2>(v);
    return v;
}

}  // namespace rie
