// quant.hip — RMSNorm + on-the-fly int8 activation quantization, and token
// embedding dequantization, for gfx950.
//
// Q8_0 (32-value blocks) follows RIE's x86 quantizer (kernels/avx2.rs:153-184):
//   amax = max|x|, d = amax/127, id = d != 0 ? 1/d : 0, q = RNE(x·id) clamped to
//   ±127, s = d·Σ(unclamped q).  Half a wavefront (32 lanes) owns one block.
// Q8_K (256-value blocks) follows quant/mod.rs:191-218: the first element with
//   the strictly largest |x| sets max, iscale = -127/max, q = round-half-away,
//   bsums over 16, d = 1/iscale.  One wavefront owns one block.
// Division and sqrt are the correctly rounded IEEE operations (no fast-math), so
// identical f32 inputs give bit-identical codes and scales.
#include "../common.hpp"
#include "../device.hpp"
#include "../kernels.hpp"
#include "../norm_quant.hpp"

namespace rie {

// Grid (row chunks, rows): every workgroup recomputes its row's sum of squares
// (the row is L2-resident) and quantizes its chunk: 16 Q8_0 blocks (two per
// wave) or 4 Q8_K blocks (one per wave).
constexpr int Q8_0_BLOCKS_PER_WG = 16;
constexpr int Q8K_BLOCKS_PER_WG = 4;

// ref_order: the norm's sum of squares in the reference's order (rms_scale_ref_wg).
template <int FMT>
__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const float *__restrict__ x, int ldx, const float *__restrict__ w,
                                                            float eps, int E, float *__restrict__ xn, ActQ8 act, int ref_order) {
    __shared__ float red[4];
    const int row = blockIdx.y;
    const float *xr = x + (size_t)row * ldx;
    const float scale = w ? (ref_order ? rms_scale_ref_wg(xr, E, eps, red) : rms_scale_wg(xr, E, eps, red)) : 1.0f;
    if (FMT == ACT_Q8_0) {
        const int b0 = blockIdx.x * Q8_0_BLOCKS_PER_WG;
        quant_q8_0_range(xr, w, scale, E, xn, act, row, b0, min(E >> 5, b0 + Q8_0_BLOCKS_PER_WG));
    } else {
        const int b0 = blockIdx.x * Q8K_BLOCKS_PER_WG;
        quant_q8k_range(xr, w, scale, E, xn, act, row, b0, min(E >> 8, b0 + Q8K_BLOCKS_PER_WG));
    }
}

// Q8_0 of whole rows, one workgroup per row: thread τ owns values 16τ..16τ+15 of
// each 4096-value pass (a 32-block is a thread pair), so every load is 16 bytes
// and every thread writes its 16 codes with one store.  With w, the row is first
// reduced to its RMSNorm scale and then quantized (second read from L2).
__global__ __launch_bounds__(256) void q8_0_rows_kernel(const float *__restrict__ x, int ldx, const float *__restrict__ w, float eps,
                                                        int E, float *__restrict__ xn, ActQ8 act, int ref_order) {
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (size_t)row * ldx;
    float scale = 1.0f;
    if (w && ref_order) {
        scale = rms_scale_ref_wg(xr, E, eps, red);
    } else if (w) {
        float ss = 0.0f;
        for (int i0 = 16 * tid; i0 < E; i0 += 4096)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 v = *(const float4 *)(xr + i0 + 4 * k);
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
            }
        ss = wave_sum(ss, 64);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)E + eps);
    }
    for (int base = 0; base < E; base += 4096) {  // uniform trip count: every thread reaches the pair exchanges
        const int i0 = base + 16 * tid;
        const bool on = i0 < E;                  // E % 32 == 0: both threads of a pair agree
        float y[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f), g = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            if (on) {
                v = *(const float4 *)(xr + i0 + 4 * k);
                if (w) g = *(const float4 *)(w + i0 + 4 * k);
            }
            y[4 * k] = w ? v.x * scale * g.x : v.x;
            y[4 * k + 1] = w ? v.y * scale * g.y : v.y;
            y[4 * k + 2] = w ? v.z * scale * g.z : v.z;
            y[4 * k + 3] = w ? v.w * scale * g.w : v.w;
        }
        if (xn && on)
#pragma unroll
            for (int k = 0; k < 4; k++) *(float4 *)(xn + (size_t)row * E + i0 + 4 * k) = make_float4(y[4 * k], y[4 * k + 1], y[4 * k + 2], y[4 * k + 3]);
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e++) amax = fmaxf(amax, fabsf(y[e]));
        amax = fmaxf(amax, xor_f<1>(amax));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t packed[4];
        int su = 0, sc = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int q = (int)rintf(y[4 * k + e] * id);
                const int qc = q < -127 ? -127 : (q > 127 ? 127 : q);
                su += q;
                sc += qc;
                word |= ((uint32_t)(qc & 0xff)) << (8 * e);
            }
            packed[k] = word;
        }
        su += xor_i<1>(su);
        sc += xor_i<1>(sc);
        if (on) {
            *(uint4 *)(act.qs + (size_t)row * E + i0) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            if ((tid & 1) == 0) {
                const size_t bi = ((size_t)row * E + i0) >> 5;
                act.d[bi] = d;
                if (act.s) act.s[bi] = d * (float)su;
                if (act.isum) act.isum[bi] = sc;
            }
        }
    }
}

void launch_rmsnorm_quant(const float *x, int ldx, const float *w, float eps, int n_rows, int E, float *xn, int fmt, const ActQ8 &act,
                          hipStream_t st, bool ref_order) {
    const int ro = ref_order ? 1 : 0;
    if (fmt == ACT_Q8_0) {
        if (E % 32 == 0 && ldx % 4 == 0) {
            hipLaunchKernelGGL(q8_0_rows_kernel, dim3(n_rows), dim3(256), 0, st, x, ldx, w, eps, E, xn, act, ro);
            return;
        }
        const int chunks = (E / 32 + Q8_0_BLOCKS_PER_WG - 1) / Q8_0_BLOCKS_PER_WG;
        hipLaunchKernelGGL(rmsnorm_quant_kernel<ACT_Q8_0>, dim3(chunks, n_rows), dim3(256), 0, st, x, ldx, w, eps, E, xn, act, ro);
    } else {
        const int chunks = (E / 256 + Q8K_BLOCKS_PER_WG - 1) / Q8K_BLOCKS_PER_WG;
        hipLaunchKernelGGL(rmsnorm_quant_kernel<ACT_Q8K>, dim3(chunks, n_rows), dim3(256), 0, st, x, ldx, w, eps, E, xn, act, ro);
    }
}

// RMSNorm without quantization (f32 out), one row per workgroup: ops.rs:7-14
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, int ldx, const float *__restrict__ w, float eps,
                                                      int E, float *__restrict__ out, int ldo, int inplace_assoc, int ref_order) {
    const int row = blockIdx.x, tid = threadIdx.x;
    const float *xr = x + (size_t)row * ldx;
    __shared__ float red[4];
    __shared__ float s_scale;
    float scale;
    if (ref_order) {
        scale = rms_scale_ref_wg(xr, E, eps, red);
    } else {
        float ss = 0.0f;
        for (int i = tid; i < E; i += 256) ss = fmaf(xr[i], xr[i], ss);
        ss = wave_sum(ss, 64);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        if (tid == 0) s_scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)E + eps);
        __syncthreads();
        scale = s_scale;
    }
    float *o = out + (size_t)row * ldo;
    for (int i = tid; i < E; i += 256) o[i] = inplace_assoc ? xr[i] * (scale * w[i]) : xr[i] * scale * w[i];
}

void launch_rmsnorm(const float *x, int ldx, const float *w, float eps, int n_rows, int E, float *out, int ldo, int inplace_assoc,
                    hipStream_t st, bool ref_order) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(n_rows), dim3(256), 0, st, x, ldx, w, eps, E, out, ldo, inplace_assoc, ref_order ? 1 : 0);
}

// ---- token embedding: dequantize_row (quant/reference.rs:53-215) ---------------
// Token ids from the host are checked there; an id made on the device (the greedy
// argmax of a row without a finite maximum gives 0x7fffffff) that is not a row of
// the table gives a NaN row instead of a read past the table.
__global__ __launch_bounds__(256) void embed_kernel(const uint32_t *__restrict__ tokens, const uint8_t *__restrict__ table, int ty,
                                                    int E, size_t rb, uint32_t n_rows, float scale, float *__restrict__ x) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= E) return;
    const uint32_t tok = tokens[t];
    if (tok >= n_rows) {
        x[(size_t)t * E + i] = __builtin_nanf("");
        return;
    }
    const uint8_t *row = table + (size_t)tok * rb;
    float y = 0.0f;
    switch (ty) {
    case T_F32: y = ((const float *)row)[i]; break;
    case T_F16: y = h2f(((const uint16_t *)row)[i]); break;
    case T_Q4_0: {
        const uint8_t *b = row + (i >> 5) * 18;
        const int j = i & 31;
        const float d = h2f(b[0] | (b[1] << 8));
        const int q = j < 16 ? (b[2 + j] & 15) : (b[2 + j - 16] >> 4);
        y = (float)(q - 8) * d;
        break;
    }
    case T_Q8_0: {
        const uint8_t *b = row + (i >> 5) * 34;
        y = (float)(int8_t)b[2 + (i & 31)] * h2f(b[0] | (b[1] << 8));
        break;
    }
    case T_BF16: y = __uint_as_float((uint32_t)((const uint16_t *)row)[i] << 16); break;
    case T_Q4_1: {
        const uint8_t *b = row + (i >> 5) * 20;
        const int j = i & 31;
        const int q = j < 16 ? (b[4 + j] & 15) : (b[4 + j - 16] >> 4);
        y = (float)q * h2f(b[0] | (b[1] << 8)) + h2f(b[2] | (b[3] << 8));
        break;
    }
    case T_Q5_0:
    case T_Q5_1: {
        const bool m = ty == T_Q5_1;
        const uint8_t *b = row + (i >> 5) * (m ? 24 : 22);
        const int j = i & 31;
        const uint8_t *hq = b + (m ? 4 : 2);
        const uint32_t qh = hq[0] | (hq[1] << 8) | (hq[2] << 16) | ((uint32_t)hq[3] << 24);
        const uint8_t *qs = hq + 4;
        const int lo = j < 16 ? (qs[j] & 15) : (qs[j - 16] >> 4);
        const int q = lo | (((qh >> j) & 1) << 4);
        const float d = h2f(b[0] | (b[1] << 8));
        y = m ? (float)q * d + h2f(b[2] | (b[3] << 8)) : (float)(q - 16) * d;
        break;
    }
    case T_Q2_K: {
        const uint8_t *b = row + (i >> 8) * 84;
        const int r = i & 255, n = r >> 7, js = (r >> 5) & 3, half = (r >> 4) & 1, l = r & 15;
        const uint8_t sc = b[8 * n + 2 * js + half];
        const int q = (b[16 + 32 * n + l + 16 * half] >> (2 * js)) & 3;
        const float d = h2f(b[80] | (b[81] << 8)), mn = h2f(b[82] | (b[83] << 8));
        y = d * (float)(sc & 0xF) * (float)q - mn * (float)(sc >> 4);
        break;
    }
    case T_Q3_K: {
        const uint8_t *b = row + (i >> 8) * 110;
        const int r = i & 255, n = r >> 7, js = (r >> 5) & 3, half = (r >> 4) & 1, l = r & 15;
        const int idx = l + 16 * half, is = 8 * n + 2 * js + half;
        const int v = ((b[32 + 32 * n + idx] >> (2 * js)) & 3) - ((b[idx] >> (4 * n + js)) & 1 ? 0 : 4);
        // 6-bit scale `is` (unpack_q3k_scales): low 4 bits from bytes 0..7, high 2 bits from bytes 8..11
        const int lo4 = is < 8 ? (b[96 + is] & 0xF) : (b[96 + is - 8] >> 4);
        const int hi2 = (b[96 + 8 + (is & 3)] >> (2 * (is >> 2))) & 3;
        const int sc = (lo4 | (hi2 << 4)) - 32;
        y = h2f(b[108] | (b[109] << 8)) * (float)sc * (float)v;
        break;
    }
    case T_Q5_K: {
        const uint8_t *b = row + (i >> 8) * 176;
        const int r = i & 255, j = r >> 6, l = r & 63;
        const float d = h2f(b[0] | (b[1] << 8)), dmin = h2f(b[2] | (b[3] << 8));
        const uint8_t *q = b + 4;
        const int sj = 2 * j + (l >= 32);
        uint8_t sc, mn;
        if (sj < 4) {
            sc = q[sj] & 63;
            mn = q[sj + 4] & 63;
        } else {
            sc = (q[sj + 4] & 0xF) | ((q[sj - 4] >> 6) << 4);
            mn = (q[sj + 4] >> 4) | ((q[sj] >> 6) << 4);
        }
        const uint8_t ql = b[48 + 32 * j + (l & 31)];
        const int hbit = (b[16 + (l & 31)] >> (2 * j + (l >= 32))) & 1;
        const int v = (l < 32 ? (ql & 15) : (ql >> 4)) + 16 * hbit;
        y = d * (float)sc * (float)v - dmin * (float)mn;
        break;
    }
    case T_Q4_K: {
        const uint8_t *b = row + (i >> 8) * 144;
        const int r = i & 255, j = r >> 6, l = r & 63;
        const float d = h2f(b[0] | (b[1] << 8)), dmin = h2f(b[2] | (b[3] << 8));
        const uint8_t *q = b + 4;
        const int sj = 2 * j + (l >= 32);
        uint8_t sc, mn;
        if (sj < 4) {
            sc = q[sj] & 63;
            mn = q[sj + 4] & 63;
        } else {
            sc = (q[sj + 4] & 0xF) | ((q[sj - 4] >> 6) << 4);
            mn = (q[sj + 4] >> 4) | ((q[sj] >> 6) << 4);
        }
        const uint8_t qb = b[16 + 32 * j + (l & 31)];
        const int v = l < 32 ? (qb & 15) : (qb >> 4);
        y = d * (float)sc * (float)v - dmin * (float)mn;
        break;
    }
    case T_Q6_K: {
        const uint8_t *b = row + (i >> 8) * 210;
        const int r = i & 255, n = r >> 7, k = (r & 127) >> 5, l = r & 31;
        const uint8_t qlb = b[64 * n + l + 32 * (k & 1)];
        const uint8_t qhb = b[128 + 32 * n + l];
        const int q = (((k >= 2) ? (qlb >> 4) : (qlb & 15)) | (((qhb >> (2 * k)) & 3) << 4)) - 32;
        const float d = h2f(b[208] | (b[209] << 8));
        y = d * (float)(int8_t)b[192 + 8 * n + 2 * k + (l >> 4)] * (float)q;
        break;
    }
    default: break;
    }
    if (scale != 1.0f) y *= scale;
    x[(size_t)t * E + i] = y;
}

void launch_embed(const uint32_t *tokens, int n, const DevWeight &table, float scale, float *x, hipStream_t st) {
    const int E = (int)table.cols;
    hipLaunchKernelGGL(embed_kernel, dim3((E + 255) / 256, n), dim3(256), 0, st, tokens, table.data, table.ty, E, table.rb(),
                       (uint32_t)table.rows, scale, x);
}

}  // namespace rie
