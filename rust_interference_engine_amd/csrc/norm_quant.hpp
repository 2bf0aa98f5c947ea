// norm_quant.hpp — RMSNorm of one row and its int8 activation quantization, as
// workgroup-level device functions (the standalone kernel in quant.hip).
//
// RMSNorm: y = x·(1/√(Σx²/E + eps))·w  (ops.rs:7-14).
// Q8_0 (kernels/avx2.rs:153-184): amax, d = amax/127, id = d≠0 ? 1/d : 0,
//   q = RNE(y·id) clamped to ±127, s = d·Σ(unclamped q); half a wave per block.
// Q8_K (quant/mod.rs:191-218): first strictly largest |y| sets max,
//   iscale = −127/max, q = round-half-away, bsums over 16, d = 1/iscale; one
//   wave per block.
#pragma once

#include "common.hpp"
#include "device.hpp"

namespace rie {

// Row reads: plain, or (COH) agent-scope loads that are coherent across the
// XCDs' L2 caches, for a row that other workgroups of the same grid wrote.
template <bool COH>
__device__ __forceinline__ float ld_row(const float *p) {
    if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}
template <bool COH>
__device__ __forceinline__ float4 ld_row4(const float *p) {
    if constexpr (COH) return make_float4(ld_row<true>(p), ld_row<true>(p + 1), ld_row<true>(p + 2), ld_row<true>(p + 3));
    else return *(const float4 *)p;
}

// 1/√(Σx²/E + eps) of a row, for a 256-thread workgroup (red: 4 floats of LDS).
template <bool COH = false>
__device__ __forceinline__ float rms_scale_wg(const float *__restrict__ xr, int E, float eps, float *red) {
    const int tid = threadIdx.x;
    float ss = 0.0f;
    for (int i = tid * 4; i < E; i += 1024) {
        const float4 v = ld_row4<COH>(xr + i);
        ss = fmaf(v.x, v.x, ss);
        ss = fmaf(v.y, v.y, ss);
        ss = fmaf(v.z, v.z, ss);
        ss = fmaf(v.w, v.w, ss);
    }
    ss = wave_sum(ss, 64);
    __syncthreads();  // red may still be read by a previous call
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float t = (red[0] + red[1]) + (red[2] + red[3]);
    return 1.0f / sqrtf(t / (float)E + eps);
}

// Σx² of a row summed in the order of the reference's x86 dot_f32
// (kernels/avx2.rs:186-203, called by rmsnorm, ops.rs:7-14): lane L < 16 of the
// calling wave accumulates x[16j+L]² with one fma per j, in j order (lanes 0-7
// are the accumulator acc0, lanes 8-15 acc1); then acc0 + acc1 and the hsum_ps
// tree ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)) as exchanges at lane offsets 8, 4,
// 2, 1 (each addition the reference's, operands commuted at most); then the
// sequential tail s + x[i]·x[i] (not fused) over the last E % 16 values.  For
// the same row this is the reference's sum bit for bit.  Serial: E/16 dependent fmas.
// 1/√(Σx²/E + eps) with Σx² in that order, for a workgroup of 256 threads (red:
// 1 float of LDS; lanes 16-63 of the first wave repeat lanes 0-15).  The
// row passes through LDS in chunks of 4096 values, one coalesced load round per
// chunk, and the first wave runs the serial fma chains from LDS.
template <bool COH = false>
__device__ __forceinline__ float rms_scale_ref_wg(const float *__restrict__ xr, int E, float eps, float *red) {
    constexpr int CH = 4096;
    __shared__ float s_chunk[CH];
    const int tid = threadIdx.x, L = tid & 15;
    const int body = (E >> 4) << 4;  // values of the 16-lane chains; the rest is the tail
    float acc = 0.0f;
    __syncthreads();  // red and s_chunk may still be read by a previous call
    for (int c0 = 0; c0 < body; c0 += CH) {
        const int cn = min(CH, body - c0);
#pragma unroll 4
        for (int i = tid; i < cn; i += 256) s_chunk[i] = ld_row<COH>(xr + c0 + i);
        __syncthreads();
        if (tid < 64) {
            const int nj = cn >> 4;
            int j = 0;
            for (; j + 8 <= nj; j += 8) {
                float v[8];
#pragma unroll
                for (int u = 0; u < 8; u++) v[u] = s_chunk[16 * (j + u) + L];
#pragma unroll
                for (int u = 0; u < 8; u++) acc = fmaf(v[u], v[u], acc);
            }
            for (; j < nj; j++) {
                const float v = s_chunk[16 * j + L];
                acc = fmaf(v, v, acc);
            }
        }
        __syncthreads();
    }
    if (tid < 64) {
        acc = acc + xor_f<8>(acc);
        acc = acc + xor_f<4>(acc);
        acc = acc + xor_f<2>(acc);
        acc = acc + xor_f<1>(acc);
        float ss = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, acc)));
        for (int i = body; i < E; i++) {
            const float v = ld_row<COH>(xr + i);
            ss = ss + v * v;
        }
        if (tid == 0) red[0] = 1.0f / sqrtf(ss / (float)E + eps);
    }
    __syncthreads();
    return red[0];
}

// Q8_0 blocks [blo, bhi) of row `row` (E values); y = w ? x·scale·w : x.
template <bool COH = false>
__device__ __forceinline__ void quant_q8_0_range(const float *__restrict__ xr, const float *__restrict__ w, float scale, int E,
                                                 float *__restrict__ xn, const ActQ8 &act, size_t row, int blo, int bhi) {
    const int tid = threadIdx.x;
    const int hw = tid >> 5, j = tid & 31;
    const int nb = E >> 5;
    for (int b = blo + hw; b < bhi; b += 8) {
        const int i = (b << 5) + j;
        const float xv = ld_row<COH>(xr + i);
        const float y = w ? xv * scale * w[i] : xv;
        if (xn) xn[row * E + i] = y;
        float amax = fabsf(y);
        amax = xmax_f<32>(amax);
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const int q = (int)rintf(y * id);
        const int qc = q < -127 ? -127 : (q > 127 ? 127 : q);
        int su = q, sc = qc;
        su = xsum_i<32>(su);
        sc = xsum_i<32>(sc);
        act.qs[row * E + i] = (int8_t)qc;
        if (j == 0) {
            const size_t bi = row * nb + b;
            act.d[bi] = d;
            if (act.s) act.s[bi] = d * (float)su;
            if (act.isum) act.isum[bi] = sc;
        }
    }
}

// Q8_K blocks [blo, bhi) of row `row`.
template <bool COH = false>
__device__ __forceinline__ void quant_q8k_range(const float *__restrict__ xr, const float *__restrict__ w, float scale, int E,
                                                float *__restrict__ xn, const ActQ8 &act, size_t row, int blo, int bhi) {
    const int tid = threadIdx.x;
    const int wv = tid >> 6, l = tid & 63;
    const int nb = E >> 8;
    for (int b = blo + wv; b < bhi; b += 4) {
        const int i0 = (b << 8) + (l << 2);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float xv = ld_row<COH>(xr + i0 + e);
            y[e] = w ? xv * scale * w[i0 + e] : xv;
            if (xn) xn[row * E + i0 + e] = y[e];
        }
        float amax = 0.0f, mx = 0.0f;
        int idx = 0x7fffffff;
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (fabsf(y[e]) > amax) {
                amax = fabsf(y[e]);
                mx = y[e];
                idx = (l << 2) + e;
            }
        xor_down<32, 1>([&](auto oc) {
            constexpr int o = decltype(oc)::value;
            const float oa = xor_f<o>(amax), om = xor_f<o>(mx);
            const int oi = xor_i<o>(idx);
            if (oa > amax || (oa == amax && oi < idx)) {
                amax = oa;
                mx = om;
                idx = oi;
            }
        });
        int8_t *qo = act.qs + row * E + i0;
        const size_t bi = row * nb + b;
        if (amax == 0.0f) {
#pragma unroll
            for (int e = 0; e < 4; e++) qo[e] = 0;
            if ((l & 3) == 0) act.bsums[row * (E >> 4) + (b << 4) + (l >> 2)] = 0;
            if (l == 0) act.d[bi] = 0.0f;
        } else {
            const float iscale = -127.0f / mx;
            int s4 = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int q = (int)roundf(iscale * y[e]);
                q = q < -127 ? -127 : (q > 127 ? 127 : q);
                qo[e] = (int8_t)q;
                s4 += q;
            }
            s4 += xor_i<1>(s4);
            s4 += xor_i<2>(s4);
            if ((l & 3) == 0) act.bsums[row * (E >> 4) + (b << 4) + (l >> 2)] = (int16_t)s4;
            if (l == 0) act.d[bi] = 1.0f / iscale;
        }
    }
}

}  // namespace rie
