// device.hpp — device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace rie {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4 ld_nt16(const void *p) { return __builtin_nontemporal_load((const u32x4 *)p); }
__device__ __forceinline__ f32x4 ld_nt16f(const void *p) { return __builtin_nontemporal_load((const f32x4 *)p); }

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
    for (int i = 0; i < 9; i++) w[i] = __builtin_nontemporal_load(q + i);
#pragma unroll
    for (int i = 0; i < 8; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float gelu_tanh_f(float x) {
    const float k = 0.7978846f;
    return 0.5f * x * (1.0f + tanhf(k * x * (1.0f + 0.044715f * x * x)));
}

}  // namespace rie
