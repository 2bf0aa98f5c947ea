// gemv.hip — decode matrix-vector products of ggml-block weights with int8
// activations (kernels/mod.rs:136-232 and quant/reference.rs:221-385 in the
// reference define the arithmetic), written for CDNA4 wavefronts.
//
// Weights stay in their native GGUF block bytes in HBM.  Each row is split into
// "units" that a lane can load with dword-aligned vector loads and reduce with
// v_dot4_i32_i8 (sdot4):
//   Q4_0 / Q8_0 : a pair of 32-blocks (36 / 68 bytes, dword aligned when K%64==0)
//   Q4_K        : one 64-value quarter of a 256-superblock (16-byte aligned)
//   Q6_K        : one 32-value eighth of a 210-byte superblock (2-byte aligned,
//                 realigned with v_alignbyte)
// LPR lanes of a wavefront share a row (64/LPR rows per wave), every weight byte
// is loaded once per launch with non-temporal loads so the streamed weights do
// not evict the activations, and a lane's partial sums are reduced across the
// LPR lanes with cross-lane shuffles.  Per-block integer dot products are exact;
// only the float accumulation order differs from the CPU path.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"

namespace rie {

constexpr int MAXT = 4;  // tokens processed per weight load
constexpr uint32_t M4 = 0x0F0F0F0Fu;

struct SegP {
    const uint8_t *w;
    size_t rb;
    int rows;
    float *out;
    int ld;
    int epi;
};

struct GemvP {
    SegP seg[3];
    int nseg;
    int total_rows;
    ActQ8 act;
    const float *actf;
    int n_tok, K;
    int glu;  // 0 none, 1 silu, 2 gelu-tanh (seg[0] = gate, seg[1] = up)
};

template <int TY>
__device__ __forceinline__ int units_per_row(int K) {
    if (TY == T_Q6_K) return K >> 5;
    if (TY == T_F32 || TY == T_F16) return K >> 3;
    return K >> 6;
}

template <int TY>
__device__ __forceinline__ void unit_dot(const uint8_t *__restrict__ row, int u, const ActQ8 &act, const float *__restrict__ actf, int K,
                                         int t0, int nt, float acc[MAXT]) {
    if constexpr (TY == T_Q4_0) {
        const uint32_t *wp = (const uint32_t *)(row + 36 * u);
        uint32_t w[9];
#pragma unroll
        for (int i = 0; i < 9; i++) w[i] = __builtin_nontemporal_load(wp + i);
        const float d0 = h2f(w[0] & 0xffff), d1 = h2f(w[4] >> 16);
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
#pragma unroll
        for (int i = 0; i < 4; i++) q[4 + i] = w[5 + i];
        const int nb = K >> 5;
#pragma unroll
        for (int tt = 0; tt < MAXT; tt++) {
            if (tt >= nt) break;
            const int t = t0 + tt;
            const uint4 *ap = (const uint4 *)(act.qs + (size_t)t * K + 64 * u);
            const uint4 a0 = ap[0], a1 = ap[1], a2 = ap[2], a3 = ap[3];
            int i0 = 0, i1 = 0;
            i0 = sdot4(q[0] & M4, a0.x, i0); i0 = sdot4(q[1] & M4, a0.y, i0);
            i0 = sdot4(q[2] & M4, a0.z, i0); i0 = sdot4(q[3] & M4, a0.w, i0);
            i0 = sdot4((q[0] >> 4) & M4, a1.x, i0); i0 = sdot4((q[1] >> 4) & M4, a1.y, i0);
            i0 = sdot4((q[2] >> 4) & M4, a1.z, i0); i0 = sdot4((q[3] >> 4) & M4, a1.w, i0);
            i1 = sdot4(q[4] & M4, a2.x, i1); i1 = sdot4(q[5] & M4, a2.y, i1);
            i1 = sdot4(q[6] & M4, a2.z, i1); i1 = sdot4(q[7] & M4, a2.w, i1);
            i1 = sdot4((q[4] >> 4) & M4, a3.x, i1); i1 = sdot4((q[5] >> 4) & M4, a3.y, i1);
            i1 = sdot4((q[6] >> 4) & M4, a3.z, i1); i1 = sdot4((q[7] >> 4) & M4, a3.w, i1);
            const size_t bi = (size_t)t * nb + 2 * u;
            i0 -= 8 * act.isum[bi];
            i1 -= 8 * act.isum[bi + 1];
            acc[tt] = fmaf(d0 * act.d[bi], (float)i0, acc[tt]);
            acc[tt] = fmaf(d1 * act.d[bi + 1], (float)i1, acc[tt]);
        }
    } else if constexpr (TY == T_Q8_0) {
        const uint32_t *wp = (const uint32_t *)(row + 68 * u);
        uint32_t w[17];
#pragma unroll
        for (int i = 0; i < 17; i++) w[i] = __builtin_nontemporal_load(wp + i);
        const float d0 = h2f(w[0] & 0xffff), d1 = h2f(w[8] >> 16);
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
        const int nb = K >> 5;
#pragma unroll
        for (int tt = 0; tt < MAXT; tt++) {
            if (tt >= nt) break;
            const int t = t0 + tt;
            const uint32_t *a = (const uint32_t *)(act.qs + (size_t)t * K + 64 * u);
            int i0 = 0, i1 = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) i0 = sdot4(q[i], a[i], i0);
#pragma unroll
            for (int i = 0; i < 8; i++) i1 = sdot4(w[9 + i], a[8 + i], i1);
            const size_t bi = (size_t)t * nb + 2 * u;
            acc[tt] = fmaf(d0 * act.d[bi], (float)i0, acc[tt]);
            acc[tt] = fmaf(d1 * act.d[bi + 1], (float)i1, acc[tt]);
        }
    } else if constexpr (TY == T_Q4_K) {
        const int sb = u >> 2, qi = u & 3;
        const uint8_t *b = row + 144 * sb;
        const u32x4 hdr = ld_nt16(b);
        const u32x4 v0 = ld_nt16(b + 16 + 32 * qi);
        const u32x4 v1 = ld_nt16(b + 32 + 32 * qi);
        const float d = h2f(hdr.x & 0xffff), dmin = h2f(hdr.x >> 16);
        uint8_t s[12];
        const uint32_t h1 = hdr.y, h2 = hdr.z, h3 = hdr.w;
        __builtin_memcpy(s, &h1, 4);
        __builtin_memcpy(s + 4, &h2, 4);
        __builtin_memcpy(s + 8, &h3, 4);
        int sc[2], mn[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int j = 2 * qi + h;
            if (j < 4) {
                sc[h] = s[j] & 63;
                mn[h] = s[j + 4] & 63;
            } else {
                sc[h] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
                mn[h] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
            }
        }
        const uint32_t v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        const int nsb = K >> 8;
#pragma unroll
        for (int tt = 0; tt < MAXT; tt++) {
            if (tt >= nt) break;
            const int t = t0 + tt;
            const uint32_t *a = (const uint32_t *)(act.qs + (size_t)t * K + 256 * sb + 64 * qi);
            int s1 = 0, s2 = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) s1 = sdot4(v[i] & M4, a[i], s1);
#pragma unroll
            for (int i = 0; i < 8; i++) s2 = sdot4((v[i] >> 4) & M4, a[8 + i], s2);
            const int16_t *bs = act.bsums + (size_t)t * (K >> 4) + 16 * sb + 4 * qi;
            const int sumi = s1 * sc[0] + s2 * sc[1];
            const int summ = mn[0] * ((int)bs[0] + bs[1]) + mn[1] * ((int)bs[2] + bs[3]);
            const float da = act.d[(size_t)t * nsb + sb];
            acc[tt] += (d * da) * (float)sumi - (dmin * da) * (float)summ;
        }
    } else if constexpr (TY == T_Q6_K) {
        const int sb = u >> 3, r = u & 7, n = r >> 2, k = r & 3;
        const uint8_t *b = row + 210 * sb;
        uint32_t ql[8], qh[8];
        load32_a2(b + 64 * n + 32 * (k & 1), ql);
        load32_a2(b + 128 + 32 * n, qh);
        const uint16_t scw = *(const uint16_t *)(b + 192 + 8 * n + 2 * k);
        const int sc_lo = (int8_t)(scw & 0xff), sc_hi = (int8_t)(scw >> 8);
        const float d = h2f(*(const uint16_t *)(b + 208));
        const int sh = k >= 2 ? 4 : 0, hs = 2 * k;
        uint32_t v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = ((ql[j] >> sh) & M4) | (((qh[j] >> hs) & 0x03030303u) << 4);
        const int nsb = K >> 8;
#pragma unroll
        for (int tt = 0; tt < MAXT; tt++) {
            if (tt >= nt) break;
            const int t = t0 + tt;
            const uint32_t *a = (const uint32_t *)(act.qs + (size_t)t * K + 256 * sb + 128 * n + 32 * k);
            int dl = 0, dh = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) dl = sdot4(v[j], a[j], dl);
#pragma unroll
            for (int j = 4; j < 8; j++) dh = sdot4(v[j], a[j], dh);
            const int16_t *bs = act.bsums + (size_t)t * (K >> 4) + 16 * sb + 8 * n + 2 * k;
            const int sumi = sc_lo * (dl - 32 * bs[0]) + sc_hi * (dh - 32 * bs[1]);
            acc[tt] = fmaf(d * act.d[(size_t)t * nsb + sb], (float)sumi, acc[tt]);
        }
    } else if constexpr (TY == T_F32) {
        const f32x4 w0 = ld_nt16f(row + 32 * u), w1 = ld_nt16f(row + 32 * u + 16);
#pragma unroll
        for (int tt = 0; tt < MAXT; tt++) {
            if (tt >= nt) break;
            const float4 *xp = (const float4 *)(actf + (size_t)(t0 + tt) * K + 8 * u);
            const float4 x0 = xp[0], x1 = xp[1];
            float s = acc[tt];
            s = fmaf(w0.x, x0.x, s); s = fmaf(w0.y, x0.y, s); s = fmaf(w0.z, x0.z, s); s = fmaf(w0.w, x0.w, s);
            s = fmaf(w1.x, x1.x, s); s = fmaf(w1.y, x1.y, s); s = fmaf(w1.z, x1.z, s); s = fmaf(w1.w, x1.w, s);
            acc[tt] = s;
        }
    } else if constexpr (TY == T_F16) {
        const u32x4 wv = ld_nt16(row + 16 * u);
        const uint32_t wd[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int tt = 0; tt < MAXT; tt++) {
            if (tt >= nt) break;
            const float *x = actf + (size_t)(t0 + tt) * K + 8 * u;
            float s = acc[tt];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                s = fmaf(h2f(wd[i] & 0xffff), x[2 * i], s);
                s = fmaf(h2f(wd[i] >> 16), x[2 * i + 1], s);
            }
            acc[tt] = s;
        }
    }
}

template <int TY, int LPR>
__global__ __launch_bounds__(256) void gemv_kernel(GemvP p) {
    constexpr int RPW = 64 / LPR;  // rows per wavefront
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, l = lane % LPR;
    const int n_waves = gridDim.x * 4;
    const int U = units_per_row<TY>(p.K);
    for (int rg = blockIdx.x * 4 + (threadIdx.x >> 6); rg * RPW < p.total_rows; rg += n_waves) {
        const int r = rg * RPW + sub;
        const bool valid = r < p.total_rows;
        // segment lookup without dynamic indexing of the kernel-argument struct
        int rr = r;
        const uint8_t *sw = p.seg[0].w;
        size_t srb = p.seg[0].rb;
        float *sout = p.seg[0].out;
        int sld = p.seg[0].ld, sepi = p.seg[0].epi;
        if (!p.glu && p.nseg > 1 && rr >= p.seg[0].rows) {
            rr -= p.seg[0].rows;
            if (p.nseg > 2 && rr >= p.seg[1].rows) {
                rr -= p.seg[1].rows;
                sw = p.seg[2].w; srb = p.seg[2].rb; sout = p.seg[2].out; sld = p.seg[2].ld; sepi = p.seg[2].epi;
            } else {
                sw = p.seg[1].w; srb = p.seg[1].rb; sout = p.seg[1].out; sld = p.seg[1].ld; sepi = p.seg[1].epi;
            }
        }
        for (int t0 = 0; t0 < p.n_tok; t0 += MAXT) {
            const int nt = min(MAXT, p.n_tok - t0);
            float acc[MAXT] = {0.f, 0.f, 0.f, 0.f};
            float acc2[MAXT] = {0.f, 0.f, 0.f, 0.f};
            if (valid) {
                const uint8_t *row = sw + (size_t)rr * srb;
                for (int u = l; u < U; u += LPR) unit_dot<TY>(row, u, p.act, p.actf, p.K, t0, nt, acc);
                if (p.glu) {
                    const uint8_t *row2 = p.seg[1].w + (size_t)rr * p.seg[1].rb;
                    for (int u = l; u < U; u += LPR) unit_dot<TY>(row2, u, p.act, p.actf, p.K, t0, nt, acc2);
                }
            }
#pragma unroll
            for (int tt = 0; tt < MAXT; tt++) {
                acc[tt] = wave_sum(acc[tt], LPR);
                if (p.glu) acc2[tt] = wave_sum(acc2[tt], LPR);
            }
            if (valid && l == 0) {
#pragma unroll
                for (int tt = 0; tt < MAXT; tt++) {
                    if (tt >= nt) break;
                    float *o = sout + (size_t)(t0 + tt) * sld + rr;
                    if (p.glu) {
                        const float g = acc[tt];
                        *o = (p.glu == 2 ? gelu_tanh_f(g) : silu_f(g)) * acc2[tt];
                    } else if (sepi == EPI_ADD) {
                        *o += acc[tt];
                    } else {
                        *o = acc[tt];
                    }
                }
            }
        }
    }
}

bool gemv_supported(int ty, size_t K) {
    switch (ty) {
    case T_Q4_0: case T_Q8_0: return K % 64 == 0;
    case T_Q4_K: case T_Q6_K: return K % 256 == 0;
    case T_F32: case T_F16: return K % 8 == 0;
    default: return false;
    }
}

template <int TY>
static void launch_t(const GemvP &p, hipStream_t st) {
    const int U = (TY == T_Q6_K) ? p.K / 32 : (TY == T_F32 || TY == T_F16) ? p.K / 8 : p.K / 64;
    int lpr = 64;
    if (U <= 8) lpr = 8;
    else if (U <= 16) lpr = 16;
    else if (U <= 32) lpr = 32;
    const int rpw = 64 / lpr;
    const int waves = (p.total_rows + rpw - 1) / rpw;
    int blocks = (waves + 3) / 4;
    if (blocks > 4096) blocks = 4096;
    switch (lpr) {
    case 8: hipLaunchKernelGGL((gemv_kernel<TY, 8>), dim3(blocks), dim3(256), 0, st, p); break;
    case 16: hipLaunchKernelGGL((gemv_kernel<TY, 16>), dim3(blocks), dim3(256), 0, st, p); break;
    case 32: hipLaunchKernelGGL((gemv_kernel<TY, 32>), dim3(blocks), dim3(256), 0, st, p); break;
    default: hipLaunchKernelGGL((gemv_kernel<TY, 64>), dim3(blocks), dim3(256), 0, st, p); break;
    }
}

static bool dispatch(int ty, const GemvP &p, hipStream_t st) {
    switch (ty) {
    case T_Q4_0: launch_t<T_Q4_0>(p, st); return true;
    case T_Q8_0: launch_t<T_Q8_0>(p, st); return true;
    case T_Q4_K: launch_t<T_Q4_K>(p, st); return true;
    case T_Q6_K: launch_t<T_Q6_K>(p, st); return true;
    case T_F32: launch_t<T_F32>(p, st); return true;
    case T_F16: launch_t<T_F16>(p, st); return true;
    default: return false;
    }
}

// The operands a weight type reads must exist: a missing activation array is a
// host-side error, never a launch.
static bool operands_ok(int ty, const ActQ8 &act, const float *act_f32) {
    switch (act_format(ty)) {
    case ACT_F32: return act_f32 != nullptr;
    case ACT_Q8_0: return act.qs && act.d && (ty != T_Q4_0 || act.isum);
    default: return act.qs && act.d && act.bsums;
    }
}

bool launch_gemv(const GemvSeg *segs, int nseg, const ActQ8 &act, const float *act_f32, int n_tok, int K, hipStream_t st) {
    if (n_tok < 1) return false;
    // segments of one launch must share a weight type; split otherwise
    int i = 0;
    while (i < nseg) {
        int j = i + 1;
        while (j < nseg && segs[j].w.ty == segs[i].w.ty) j++;
        GemvP p{};
        p.nseg = j - i;
        p.total_rows = 0;
        for (int s = i; s < j; s++) {
            if (!gemv_supported(segs[s].w.ty, K) || segs[s].w.cols != (size_t)K || !segs[s].w.data || !segs[s].out ||
                !operands_ok(segs[s].w.ty, act, act_f32))
                return false;
            p.seg[s - i] = SegP{segs[s].w.data, segs[s].w.rb(), (int)segs[s].w.rows, segs[s].out, segs[s].ld, segs[s].epi};
            p.total_rows += (int)segs[s].w.rows;
        }
        p.act = act;
        p.actf = act_f32;
        p.n_tok = n_tok;
        p.K = K;
        p.glu = 0;
        if (!dispatch(segs[i].w.ty, p, st)) return false;
        i = j;
    }
    return true;
}

bool launch_gemv_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, const float *act_f32, int n_tok, int K, float *h,
                     int ld, int gelu, hipStream_t st) {
    if (gate.ty != up.ty || gate.rows != up.rows || !gemv_supported(gate.ty, K) || gate.cols != (size_t)K || up.cols != (size_t)K ||
        !gate.data || !up.data || !h || n_tok < 1 || !operands_ok(gate.ty, act, act_f32))
        return false;
    GemvP p{};
    p.nseg = 2;
    p.seg[0] = SegP{gate.data, gate.rb(), (int)gate.rows, h, ld, EPI_STORE};
    p.seg[1] = SegP{up.data, up.rb(), (int)up.rows, h, ld, EPI_STORE};
    p.total_rows = (int)gate.rows;
    p.act = act;
    p.actf = act_f32;
    p.n_tok = n_tok;
    p.K = K;
    p.glu = gelu ? 2 : 1;
    return dispatch(gate.ty, p, st);
}

}  // namespace rie
