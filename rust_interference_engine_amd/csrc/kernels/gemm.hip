// gemm.hip — prompt-batch GEMM on int8 MFMA (placeholder until the MFMA kernel lands).
#include "../common.hpp"
#include "../kernels.hpp"

namespace rie {

bool gemm_supported(int ty, size_t K) {
    (void)ty;
    (void)K;
    return false;
}

bool launch_gemm(const GemvSeg *segs, int nseg, const ActQ8 &act, int n_tok, int K, hipStream_t st) {
    (void)segs; (void)nseg; (void)act; (void)n_tok; (void)K; (void)st;
    return false;
}

bool launch_gemm_glu(const DevWeight &gate, const DevWeight &up, const ActQ8 &act, int n_tok, int K, float *h, int ld, int gelu,
                     float *scratch, hipStream_t st) {
    (void)gate; (void)up; (void)act; (void)n_tok; (void)K; (void)h; (void)ld; (void)gelu; (void)scratch; (void)st;
    return false;
}

}  // namespace rie
