// device.hpp — device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>
#include <type_traits>

namespace rie {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));


// Weight-stream loads.  Plain loads: on gfx950 the nontemporal form measured
// about 35% slower for the decode GEMVs.
template <class T>
__device__ __forceinline__ T wload(const T *p) {
    return *p;
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

// Value held by lane (this lane xor OFF): a DPP quad permutation for OFF = 1, 2
// (VALU), one ds_swizzle (bitmask mode, within a 32-lane half) for OFF = 4..16,
// one ds_bpermute for OFF = 32; no per-call lane-id arithmetic.  Call with the
// source lanes active.
template <int OFF>
__device__ __forceinline__ int xor_i(int v) {
    static_assert(OFF == 1 || OFF == 2 || OFF == 4 || OFF == 8 || OFF == 16 || OFF == 32, "lane offset");
    if constexpr (OFF == 1) return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    else if constexpr (OFF == 2) return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    else if constexpr (OFF == 32) return __builtin_amdgcn_ds_bpermute((int)((__lane_id() ^ 32u) << 2), v);
    else return __builtin_amdgcn_ds_swizzle(v, 0x1F | (OFF << 10));
}
template <int OFF>
__device__ __forceinline__ float xor_f(float v) { return __int_as_float(xor_i<OFF>(__float_as_int(v))); }

// Both values of the lane pair {l & ~OFF, l | OFF} (OFF = 16 or 32), in both lanes of
// the pair: lo = v[l & ~OFF], hi = v[l | OFF].  One v_permlane16_swap /
// v_permlane32_swap (VALU, no LDS).  A symmetric merge written as f(lo, hi) gives
// both lanes the same bits, which are those of f(own, other) up to the order of
// commutative operations.
template <int OFF>
__device__ __forceinline__ void pair_f(float v, float &lo, float &hi) {
    static_assert(OFF == 16 || OFF == 32, "lane offset");
    const unsigned iv = __float_as_uint(v);
    if constexpr (OFF == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    }
}

// f(std::integral_constant<int, O>) for O = FROM, FROM/2, …, TO, or (xor_up) for
// O = FROM, 2·FROM, …, TO: lane-offset loops whose offsets are template arguments.
template <int FROM, int TO, class F>
__device__ __forceinline__ void xor_down(F &&f) {
    if constexpr (FROM >= TO && FROM >= 1) {
        f(std::integral_constant<int, FROM>{});
        xor_down<FROM / 2, TO>(f);
    }
}
template <int FROM, int TO, class F>
__device__ __forceinline__ void xor_up(F &&f) {
    if constexpr (FROM <= TO) {
        f(std::integral_constant<int, FROM>{});
        xor_up<FROM * 2, TO>(f);
    }
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

// Reductions over aligned groups of W lanes (W = 2..64, a power of two); every
// lane of the group receives the same result.  Within a 16-lane row: DPP quad
// exchanges, the 8-lane half mirror and the 8-lane row rotation (VALU, no LDS);
// across rows: readlane of the row results, combined in a fixed order.  The
// partner lanes are the group's own, so the group must be active.
template <int W, class T, class Op>
__device__ __forceinline__ T xreduce(T v, Op op) {
    static_assert(W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "group width");
    auto dpp = [](T x, auto ctrl) {
        if constexpr (sizeof(T) == 4 && std::is_same_v<T, float>) return dpp_f<decltype(ctrl)::value>(x);
        else return dpp_i<decltype(ctrl)::value>(x);
    };
    v = op(v, dpp(v, std::integral_constant<int, DPP_QUAD_XOR1>{}));
    if constexpr (W >= 4) v = op(v, dpp(v, std::integral_constant<int, DPP_QUAD_XOR2>{}));
    if constexpr (W >= 8) v = op(v, dpp(v, std::integral_constant<int, DPP_HALF_MIRROR>{}));
    if constexpr (W >= 16) v = op(v, dpp(v, std::integral_constant<int, DPP_ROW_ROR8>{}));
    if constexpr (W >= 32) {
        auto rl = [&](int ln) {
            if constexpr (std::is_same_v<T, float>) return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), ln));
            else return (T)__builtin_amdgcn_readlane((int)v, ln);
        };
        const T r0 = rl(0), r1 = rl(16), r2 = rl(32), r3 = rl(48);
        if constexpr (W == 32) v = (__lane_id() < 32) ? op(r0, r1) : op(r2, r3);
        else v = op(op(r0, r1), op(r2, r3));
    }
    return v;
}
template <int W>
__device__ __forceinline__ float xsum_f(float v) {
    return xreduce<W>(v, [](float a, float b) { return a + b; });
}
template <int W>
__device__ __forceinline__ int xsum_i(int v) {
    return xreduce<W>(v, [](int a, int b) { return a + b; });
}
template <int W>
__device__ __forceinline__ float xmax_f(float v) {
    return xreduce<W>(v, [](float a, float b) { return fmaxf(a, b); });
}

__device__ __forceinline__ float wave_sum(float v, int width) {
    return width >= 64 ? xsum_f<64>(v) : width >= 32 ? xsum_f<32>(v) : width >= 16 ? xsum_f<16>(v) : width >= 8 ? xsum_f<8>(v)
         : width >= 4 ? xsum_f<4>(v) : width >= 2 ? xsum_f<2>(v) : v;
}

__device__ __forceinline__ int wave_sum_i(int v, int width) {
    return width >= 64 ? xsum_i<64>(v) : width >= 32 ? xsum_i<32>(v) : width >= 16 ? xsum_i<16>(v) : width >= 8 ? xsum_i<8>(v)
         : width >= 4 ? xsum_i<4>(v) : width >= 2 ? xsum_i<2>(v) : v;
}

__device__ __forceinline__ float wave_max(float v, int width) {
    return width >= 64 ? xmax_f<64>(v) : width >= 32 ? xmax_f<32>(v) : width >= 16 ? xmax_f<16>(v) : width >= 8 ? xmax_f<8>(v)
         : width >= 4 ? xmax_f<4>(v) : width >= 2 ? xmax_f<2>(v) : v;
}

// 2^x by the hardware exponential (v_exp_f32): exp2(-inf) = 0
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr float LOG2E_F = 1.44269504088896340736f;
constexpr float LN2_F = 0.69314718055994530942f;

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
    if constexpr (W == 32) v += xor_f<16>(v);
    return v;
}
// exact integer sum over the 4 lanes of a quad
__device__ __forceinline__ int quad_sum_i(int v) {
    v += dpp_i<DPP_QUAD_XOR1>(v);
    v += dpp_i<DPP_QUAD_XOR2>(v);
    return v;
}

// Agent-coherent accesses: a relaxed agent-scope store writes through to the
// device coherence point and a relaxed agent-scope load reads from it, so data
// passed between workgroups on different XCDs needs no L2 write-back or
// invalidate.
__device__ __forceinline__ void st_coh(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float ld_coh(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// Waits until this wave's outstanding vector memory operations, stores included,
// have completed (s_waitcnt vmcnt(0); expcnt and lgkmcnt left at their maxima in
// the gfx9 encoding).  After st_coh stores this makes them visible device-wide.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Orders one wavefront's LDS accesses across its lanes (a wave's LDS operations
// execute in issue order; the fences stop the compiler from moving accesses
// across this point).  For code run by a single wave of a larger workgroup.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier for LDS data only: the fences cover the local address space,
// so it waits for the wave's LDS operations (lgkmcnt) and not for its outstanding
// global loads, which __syncthreads() (a fence on every address space) waits for.
// Arrival counts in LDS for a subset of a workgroup's waves (no s_barrier, so
// waves outside the subset need not get there): lds_arrive publishes the wave's
// earlier LDS writes (lane 0 adds one), lds_wait_count spins until n arrivals and
// orders the wave's later LDS reads after them.  The fences cover LDS only, so
// neither waits for the wave's outstanding global loads.
__device__ __forceinline__ void lds_arrive(int *cnt) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_wait_count(int *cnt, int n) {
    while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < n) __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace rie
