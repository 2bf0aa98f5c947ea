// misc.hip — greedy argmax, elementwise epilogues and MoE routing for gfx950.
#include "../common.hpp"
#include "../device.hpp"
#include "../moe_route.hpp"
#include "../kernels.hpp"

#include <algorithm>
#include <mutex>
#include <string>

namespace rie {

// sampler.rs:199-209: the first index holding the strict maximum.  NaN never wins.
__device__ __forceinline__ void amax_merge(float &v, int &i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__global__ __launch_bounds__(256) void argmax_stage1(const float *__restrict__ x, int n, int *pidx, float *pval) {
    const int tid = threadIdx.x;
    const int per = (n + gridDim.x - 1) / gridDim.x;
    const int a = blockIdx.x * per, b = min(n, a + per);
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = a + tid; i < b; i += 256) {
        const float xv = x[i];
        if (xv > v) {  // first hit within this lane's strided scan is the smallest index
            v = xv;
            idx = i;
        }
    }
    xor_down<32, 1>([&](auto o) { amax_merge(v, idx, xor_f<decltype(o)::value>(v), xor_i<decltype(o)::value>(idx)); });
    __shared__ float sv[4];
    __shared__ int si[4];
    if ((tid & 63) == 0) {
        sv[tid >> 6] = v;
        si[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; w++) amax_merge(v, idx, sv[w], si[w]);
        pval[blockIdx.x] = v;
        pidx[blockIdx.x] = idx;
    }
}

// gen != nullptr (greedy steps replayed in a graph): the token is also stored at
// gen[step[1] + 1] (below gen_cap), and the position step[0] and index step[1]
// advance by one for the next step.
__global__ __launch_bounds__(64) void argmax_stage2(const int *pidx, const float *pval, int n_part, uint32_t *out, uint32_t *gen, int *step,
                                                    int gen_cap) {
    const int tid = threadIdx.x;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = tid; i < n_part; i += 64) amax_merge(v, idx, pval[i], pidx[i]);
    xor_down<32, 1>([&](auto o) { amax_merge(v, idx, xor_f<decltype(o)::value>(v), xor_i<decltype(o)::value>(idx)); });
    if (tid == 0) {
        const uint32_t t = idx == 0x7fffffff ? 0u : (uint32_t)idx;
        *out = t;
        if (gen) {
            const int g = step[1] + 1;
            if (g < gen_cap) gen[g] = t;
            step[1] = g;
            step[0] += 1;
        }
    }
}

// Both stages in one launch: every workgroup stores its partial with agent-scope
// atomic stores (written through to the device coherence point), waits for their
// completion, and counts its arrival with a relaxed agent-scope add; the last
// workgroup to arrive re-arms the counter and reduces the partials in its first
// wave with agent-scope atomic loads, in partial order (the first strict maximum,
// as argmax_stage2).  No release or acquire, which would write back or invalidate
// the whole L2 of the XCD.
__global__ __launch_bounds__(256) void argmax_one_kernel(const float *__restrict__ x, int n, int *pidx, float *pval, int *cnt, uint32_t *out,
                                                         uint32_t *gen, int *step, int gen_cap) {
    const int tid = threadIdx.x;
    const int per = (n + gridDim.x - 1) / gridDim.x;
    const int a = blockIdx.x * per, b = min(n, a + per);
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = a + tid; i < b; i += 256) {
        const float xv = x[i];
        if (xv > v) {
            v = xv;
            idx = i;
        }
    }
    xor_down<32, 1>([&](auto o) { amax_merge(v, idx, xor_f<decltype(o)::value>(v), xor_i<decltype(o)::value>(idx)); });
    __shared__ float sv[4];
    __shared__ int si[4];
    __shared__ int s_last;
    if ((tid & 63) == 0) {
        sv[tid >> 6] = v;
        si[tid >> 6] = idx;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; w++) amax_merge(v, idx, sv[w], si[w]);
        st_coh(pval + blockIdx.x, v);
        __hip_atomic_store(pidx + blockIdx.x, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wait_vmem();
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == (int)gridDim.x - 1;
        if (s_last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last || tid >= 64) return;
    v = -INFINITY;
    idx = 0x7fffffff;
    for (int i = tid; i < (int)gridDim.x; i += 64)
        amax_merge(v, idx, ld_coh(pval + i), __hip_atomic_load(pidx + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    xor_down<32, 1>([&](auto o) { amax_merge(v, idx, xor_f<decltype(o)::value>(v), xor_i<decltype(o)::value>(idx)); });
    if (tid == 0) {
        const uint32_t t = idx == 0x7fffffff ? 0u : (uint32_t)idx;
        *out = t;
        if (gen) {
            const int g = step[1] + 1;
            if (g < gen_cap) gen[g] = t;
            step[1] = g;
            step[0] += 1;
        }
    }
}

void launch_argmax(const float *x, int n, int *partial_idx, float *partial_val, int n_part, uint32_t *out_idx, hipStream_t st, int *cnt) {
    if (cnt) {
        hipLaunchKernelGGL(argmax_one_kernel, dim3(n_part), dim3(256), 0, st, x, n, partial_idx, partial_val, cnt, out_idx, nullptr, nullptr, 0);
        return;
    }
    hipLaunchKernelGGL(argmax_stage1, dim3(n_part), dim3(256), 0, st, x, n, partial_idx, partial_val);
    hipLaunchKernelGGL(argmax_stage2, dim3(1), dim3(64), 0, st, partial_idx, partial_val, n_part, out_idx, nullptr, nullptr, 0);
}

void launch_argmax_step(const float *x, int n, int *partial_idx, float *partial_val, int n_part, uint32_t *out_idx, uint32_t *gen,
                        int *step, int gen_cap, hipStream_t st, int *cnt) {
    if (cnt) {
        hipLaunchKernelGGL(argmax_one_kernel, dim3(n_part), dim3(256), 0, st, x, n, partial_idx, partial_val, cnt, out_idx, gen, step, gen_cap);
        return;
    }
    hipLaunchKernelGGL(argmax_stage1, dim3(n_part), dim3(256), 0, st, x, n, partial_idx, partial_val);
    hipLaunchKernelGGL(argmax_stage2, dim3(1), dim3(64), 0, st, partial_idx, partial_val, n_part, out_idx, gen, step, gen_cap);
}

// ---- argmax without device allocation ----
// The partial maxima live in one fixed array of the library's static device
// memory: ARGMAX_SCRATCH_PARTS (index, value) pairs, [idx × PARTS][val × PARTS].
// Each GPU holds its own copy of the array until the process ends; the host
// never uses the symbol itself as an address, only the per-device address that
// hipGetSymbolAddress returns for it.  Nothing in it must start at zero: stage 1
// writes every partial that stage 2 reads.
static __device__ __align__(256) unsigned char scratch[ARGMAX_SCRATCH_PARTS * 8];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void *scratch_dev[MAX_DEVICES];  // device address of `scratch` on each GPU, looked up once

void *scratch_for_current_device() {
    int dev = -1;
    RIE_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEVICES) throw Error{E_RUNTIME, "device ordinal " + std::to_string(dev) + " out of range"};
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw Error{E_RUNTIME, std::string("hipGetSymbolAddress of the argmax scratch array failed: ") + hipGetErrorString(e)};
        scratch_dev[dev] = p;
    }
    return scratch_dev[dev];
}
}  // namespace

void launch_argmax_noalloc(const float *x, int n, uint32_t *out_idx, hipStream_t st) {
    if (n < 1 || n > ARGMAX_SCRATCH_PARTS * ARGMAX_SCRATCH_PER_PART)
        throw Error{E_RUNTIME, "argmax without allocation: " + std::to_string(n) + " values is outside 1.." +
                                   std::to_string(ARGMAX_SCRATCH_PARTS * ARGMAX_SCRATCH_PER_PART) + " (the scratch holds " +
                                   std::to_string(ARGMAX_SCRATCH_PARTS) + " partials of up to " +
                                   std::to_string(ARGMAX_SCRATCH_PER_PART) + " values)"};
    unsigned char *base = (unsigned char *)scratch_for_current_device();
    const int n_part = (n + ARGMAX_SCRATCH_PER_PART - 1) / ARGMAX_SCRATCH_PER_PART;
    launch_argmax(x, n, (int *)base, (float *)(base + ARGMAX_SCRATCH_PARTS * 4), n_part, out_idx, st);
}

__global__ void add_kernel(float *x, const float *y, size_t n, float scale) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = scale == 1.0f ? x[i] + y[i] : x[i] + y[i] * scale;
}

void launch_add_inplace(float *x, const float *y, size_t n, float scale, hipStream_t st) {
    hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, y, n, scale);
}

__global__ void div_kernel(float *x, size_t n, float div) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] /= div;
}

void launch_scale(float *x, size_t n, float div, hipStream_t st) {
    hipLaunchKernelGGL(div_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, div);
}

__global__ void set_int_kernel(int *p, int v) { *p = v; }

void launch_set_int(int *p, int v, hipStream_t st) { hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, st, p, v); }

__global__ void softcap_kernel(float *x, size_t n, float cap) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = cap * tanhf(x[i] / cap);
}

void launch_softcap(float *x, size_t n, float cap, hipStream_t st) {
    hipLaunchKernelGGL(softcap_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, cap);
}

void launch_quant_only(const float *x, int ldx, int n_rows, int K, int fmt, const ActQ8 &act, hipStream_t st) {
    launch_rmsnorm_quant(x, ldx, nullptr, 0.0f, n_rows, K, nullptr, fmt, act, st);
}

// MoE routing: one wavefront per token (moe_route_wave, moe_route.hpp)
__global__ __launch_bounds__(64) void moe_route_kernel(const float *logits, int n_exp, int k, int norm_topk, int unit_weights, int *sel,
                                                       float *wgt) {
    const size_t t = blockIdx.x;
    moe_route_wave(logits + t * n_exp, n_exp, k, norm_topk, unit_weights, sel + t * k, wgt + t * k);
}

// out[t] (= or +=) Σ_j w[t][j]·y[t·k + j], j in ascending expert order, starting from 0
__global__ void moe_combine_kernel(const float *__restrict__ y, const float *__restrict__ w, int k, int E, float *__restrict__ out,
                                   int epi) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= E) return;
    float o = 0.0f;
    for (int j = 0; j < k; j++) o += w[(size_t)t * k + j] * y[((size_t)t * k + j) * E + i];
    if (epi == EPI_ADD) out[(size_t)t * E + i] += o;
    else out[(size_t)t * E + i] = o;
}

void launch_moe_combine(const float *y, const float *w, int n_tok, int k, int E, float *out, int epi, hipStream_t st) {
    hipLaunchKernelGGL(moe_combine_kernel, dim3((E + 255) / 256, n_tok), dim3(256), 0, st, y, w, k, E, out, epi);
}

// xg[i] = x[rows[i]]  (rows of E floats)
__global__ void moe_gather_kernel(const float *__restrict__ x, const int *__restrict__ rows, int E, float *__restrict__ xg) {
    const int r = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i < E) xg[(size_t)r * E + i] = x[(size_t)rows[r] * E + i];
}

void launch_moe_gather(const float *x, const int *rows, int n, int E, float *xg, hipStream_t st) {
    hipLaunchKernelGGL(moe_gather_kernel, dim3((E + 255) / 256, n), dim3(256), 0, st, x, rows, E, xg);
}

// out[rows[i]] += w[i]·yg[i]; one expert's rows are distinct tokens, so no two
// threads of a launch touch the same element
__global__ void moe_scatter_add_kernel(const float *__restrict__ yg, const int *__restrict__ rows, const float *__restrict__ w, int E,
                                       float *__restrict__ out) {
    const int r = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i < E) out[(size_t)rows[r] * E + i] += w[r] * yg[(size_t)r * E + i];
}

void launch_moe_scatter_add(const float *yg, const int *rows, const float *w, int n, int E, float *out, hipStream_t st) {
    hipLaunchKernelGGL(moe_scatter_add_kernel, dim3((E + 255) / 256, n), dim3(256), 0, st, yg, rows, w, E, out);
}

// out[t] += sigmoid(g·x[t])·ys[t] (shared expert gate, cpu.rs:516-522); g may be null (scale 1)
__global__ __launch_bounds__(256) void moe_shared_add_kernel(const float *__restrict__ ys, const float *__restrict__ g,
                                                             const float *__restrict__ x, int E, float *__restrict__ out) {
    const int t = blockIdx.x, tid = threadIdx.x;
    __shared__ float red[4];
    __shared__ float s_scale;
    if (g) {
        float s = 0.0f;
        for (int i = tid; i < E; i += 256) s = fmaf(g[i], x[(size_t)t * E + i], s);
        s = wave_sum(s, 64);
        if ((tid & 63) == 0) red[tid >> 6] = s;
        __syncthreads();
        if (tid == 0) s_scale = 1.0f / (1.0f + expf(-((red[0] + red[1]) + (red[2] + red[3]))));
        __syncthreads();
    } else if (tid == 0) {
        s_scale = 1.0f;
    }
    __syncthreads();
    const float sc = s_scale;
    for (int i = tid; i < E; i += 256) out[(size_t)t * E + i] += sc * ys[(size_t)t * E + i];
}

void launch_moe_shared_add(const float *ys, const float *gate_inp, const float *x, int n_tok, int E, float *out, hipStream_t st) {
    hipLaunchKernelGGL(moe_shared_add_kernel, dim3(n_tok), dim3(256), 0, st, ys, gate_inp, x, E, out);
}

// Grouping of a prompt batch's routed pairs by expert (the assign lists of
// moe_ffn, cpu.rs:489-501), on the device: counts, their exclusive prefix, each
// pair's gathered row, and the token tiles of every expert.  Within an expert the
// rows follow the arrival order of an LDS counter: any order gives the same
// results, since a row's values depend on its own token only, and the combine sums
// each token's experts in ascending order from the pair index.  Expert ids outside
// [0, n_exp) (only from non-finite router logits) are dropped.
__global__ __launch_bounds__(1024) void moe_group_kernel(const int *__restrict__ sel, int n_pairs, int k, int n_exp, int *off,
                                                         int *row_tok, int *row_slot, int *tile_e, int *tile_r0, int *n_tiles, int bn) {
    __shared__ int cnt[512], fill[512], base[513], tbase[513];
    const int tid = threadIdx.x;
    for (int e = tid; e < n_exp; e += 1024) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    __syncthreads();
    for (int a = tid; a < n_pairs; a += 1024) {
        const int e = sel[a];
        if ((unsigned)e < (unsigned)n_exp) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int acc = 0, tacc = 0;
        for (int e = 0; e < n_exp; e++) {
            base[e] = acc;
            tbase[e] = tacc;
            acc += cnt[e];
            tacc += (cnt[e] + bn - 1) / bn;
        }
        base[n_exp] = acc;
        tbase[n_exp] = tacc;
        *n_tiles = tacc;
    }
    __syncthreads();
    for (int e = tid; e <= n_exp; e += 1024) off[e] = base[e];
    for (int a = tid; a < n_pairs; a += 1024) {
        const int e = sel[a];
        if ((unsigned)e >= (unsigned)n_exp) continue;
        const int r = base[e] + atomicAdd(&fill[e], 1);
        row_tok[r] = a / k;
        row_slot[r] = a;
    }
    for (int e = tid; e < n_exp; e += 1024)
        for (int i = 0; i < tbase[e + 1] - tbase[e]; i++) {
            tile_e[tbase[e] + i] = e;
            tile_r0[tbase[e] + i] = base[e] + i * bn;
        }
}

int moe_group_max_tiles(int n_tok, int k, int n_exp, int bn) {
    // the full tiles of all pairs, plus at most one partial tile per expert that has rows
    const int pairs = n_tok * k;
    return (pairs + bn - 1) / bn + std::min(n_exp, pairs);
}

void launch_moe_group(const int *sel, int n_tok, int k, int n_exp, int *off, int *row_tok, int *row_slot, int *tile_e, int *tile_r0,
                      int *n_tiles, int bn, hipStream_t st) {
    hipLaunchKernelGGL(moe_group_kernel, dim3(1), dim3(1024), 0, st, sel, n_tok * k, k, n_exp, off, row_tok, row_slot, tile_e, tile_r0,
                       n_tiles, bn);
}

void launch_moe_route(const float *logits, int n_tok, int n_exp, int k, int norm_topk, int unit_weights, int *sel, float *wgt,
                      hipStream_t st) {
    hipLaunchKernelGGL(moe_route_kernel, dim3(n_tok), dim3(64), 0, st, logits, n_exp, k, norm_topk, unit_weights, sel, wgt);
}

}  // namespace rie
