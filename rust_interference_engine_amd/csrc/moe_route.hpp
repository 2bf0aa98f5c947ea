// moe_route.hpp — top-k expert routing of one token by one wavefront, shared by
// the routing kernel and the router GEMV's last workgroup.
#pragma once

#include "device.hpp"

namespace rie {

// MoE routing (model/cpu.rs:487-501): softmax over the router logits, sort by
// probability descending with the lower expert index first on ties, keep the
// top k, optionally renormalize by their sum taken in sorted order.
// One wave per token: lane l holds experts l + 64i (n_exp ≤ 512, checked by the
// host).  The softmax sum runs over the experts in order, sequentially, like the
// reference's (ops.rs:38-49): one chain of adds over readlane values.  Top-k is k rounds:
// the maximum of the experts not yet taken (DPP within 16-lane rows, then the
// four row maxima), and of the experts holding it the lowest index (ballots in
// expert order), which is the reference's index tie-break (cpu.rs:495).  Lane j
// keeps the j-th choice and writes it at its rank in ascending expert order (the
// CPU path adds the experts' outputs in that order, cpu.rs:502-513, and so does
// launch_moe_combine).
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_XOR2>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_ROR4>(v));
    return fmaxf(v, dpp_f<DPP_ROW_ROR8>(v));
}
// e^x rounded once to f32: the double-precision exponential is far more accurate
// than the half-ulp f32 rounding, so this is glibc's expf (the reference's f32::exp,
// within 0.502 ulp of e^x) but for inputs within ~0.002 ulp of a rounding midpoint,
// also through the subnormal range, where the device's f32 exponential flushes e^x
// near 2^-149 to zero.
__device__ __forceinline__ float exp_f32_rn(float x) { return (float)exp((double)x); }

// One wavefront routes one token: l holds its n_exp logits; sel/wgt receive its k
// choices in ascending expert order.  NE = experts per lane (n_exp ≤ 64·NE).
// COH: the logits were published by other workgroups of the same launch with
// agent-scope atomic stores, so they are read with agent-scope atomic loads.
template <int NE, bool COH>
__device__ __forceinline__ void moe_route_wave_t(const float *l, int n_exp, int k, int norm_topk, int unit_weights, int *sel, float *wgt) {
    const int lane = threadIdx.x & 63;
    float pr[NE];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NE; i++) {
        const int e = lane + 64 * i;
        pr[i] = e < n_exp ? (COH ? ld_coh(l + e) : l[e]) : -INFINITY;
        mx = fmaxf(mx, pr[i]);
    }
    mx = wave_max(mx, 64);
    // The reference ranks the f32 probabilities as they round (ties by index), so a
    // token whose k-th place lies in the subnormal range (a peaked softmax: fewer
    // than k probabilities safely normal after the division by the sum ≤ 128) takes
    // its experts by how e^x rounds there; that wave computes its exponentials
    // again, rounded once from double (exp_f32_rn).  Elsewhere the f32 exponential
    // decides as before.
    float xs[NE];
    int normal = 0;
#pragma unroll
    for (int i = 0; i < NE; i++) {
        xs[i] = pr[i] - mx;
        pr[i] = lane + 64 * i < n_exp ? expf(xs[i]) : 0.0f;
        normal += __popcll(__ballot(pr[i] >= 0x1p-120f));
    }
    if (normal < k) {
#pragma unroll
        for (int i = 0; i < NE; i++) pr[i] = lane + 64 * i < n_exp ? exp_f32_rn(xs[i]) : 0.0f;
    }
    // the sum over the experts in order, one add at a time (expert e sits in lane
    // e mod 64, register e / 64): the same chain in every lane, through readlane;
    // the zeros past n_exp add nothing
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NE; i++)
#pragma unroll
        for (int ln = 0; ln < 64; ln++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr[i]), ln));
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < NE; i++) pr[i] *= inv;
    uint32_t taken = 0;  // bit i: expert lane + 64i is chosen
    int my_c = 0x7fffffff;
    float my_v = 0.0f, norm = 0.0f;
    for (int j = 0; j < k; j++) {
        float v = -INFINITY;
#pragma unroll
        for (int i = 0; i < NE; i++)
            if (lane + 64 * i < n_exp && !((taken >> i) & 1u)) v = fmaxf(v, pr[i]);
        v = row_max16(v);
        const auto rl = [&](int ln) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), ln)); };
        float m = fmaxf(fmaxf(rl(0), rl(16)), fmaxf(rl(32), rl(48)));  // the row maxima
        int idx = 0x7fffffff;
#pragma unroll
        for (int i = NE - 1; i >= 0; i--) {  // the lowest expert index holding m
            const bool cand = lane + 64 * i < n_exp && !((taken >> i) & 1u) && pr[i] == m;
            const uint64_t b = __ballot(cand);
            if (b) idx = 64 * i + __builtin_ctzll(b);
        }
        if (idx == 0x7fffffff) {
            // No expert left holds a number: the probabilities are NaN (a NaN or
            // +Inf logit, or every logit -Inf, makes the softmax sum NaN).  The
            // reference's comparator calls NaN pairs Equal and falls back to the
            // index (cpu.rs:495), so the lowest untaken expert comes next, with
            // its NaN probability.
#pragma unroll
            for (int i = NE - 1; i >= 0; i--) {
                const uint64_t b = __ballot(lane + 64 * i < n_exp && !((taken >> i) & 1u));
                if (b) idx = 64 * i + __builtin_ctzll(b);
            }
            float pv = pr[0];
#pragma unroll
            for (int i = 1; i < NE; i++)
                if ((idx >> 6) == i) pv = pr[i];
            m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pv), idx & 63));
        }
        if (idx < n_exp && (idx & 63) == lane) taken |= 1u << (idx >> 6);
        if (lane == j) {
            my_c = idx;
            my_v = m;
        }
        norm += m;  // in choice order
    }
    if (!norm_topk) norm = 1.0f;
    int rank = 0;
    for (int q = 0; q < k; q++) rank += __builtin_amdgcn_readlane(my_c, q) < my_c;
    if (lane < k) {
        sel[rank] = my_c;
        wgt[rank] = unit_weights ? 1.0f : my_v / norm;
    }
}
template <bool COH = false>
__device__ __forceinline__ void moe_route_wave(const float *l, int n_exp, int k, int norm_topk, int unit_weights, int *sel, float *wgt) {
    if (n_exp <= 64) moe_route_wave_t<1, COH>(l, n_exp, k, norm_topk, unit_weights, sel, wgt);
    else if (n_exp <= 128) moe_route_wave_t<2, COH>(l, n_exp, k, norm_topk, unit_weights, sel, wgt);
    else if (n_exp <= 256) moe_route_wave_t<4, COH>(l, n_exp, k, norm_topk, unit_weights, sel, wgt);
    else moe_route_wave_t<8, COH>(l, n_exp, k, norm_topk, unit_weights, sel, wgt);
}


}  // namespace rie
