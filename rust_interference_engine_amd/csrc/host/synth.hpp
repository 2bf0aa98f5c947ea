// synth.hpp — synthetic GGUF images (the workload generator behind
// `rie bench --synthetic`, crates/rie-core/src/testing.rs in the reference).
#pragma once

#include "../../../include/rie_hip.h"

#include <cstdint>
#include <vector>

namespace rie {

int32_t synth_tiny(const char *arch, int32_t wtype, rie_hip_synth_spec *out);
int32_t synth_preset(const char *name, int32_t wtype, rie_hip_synth_spec *out);
// returns a malloc'd GGUF image (release with free) and its size
uint8_t *synth_build(const rie_hip_synth_spec &spec, int n_threads, size_t *out_len);
// the workload generator's weight quantizers (Q4_0, Q8_0, Q4_K, Q6_K) on n values
bool synth_quantize(int ty, const float *x, size_t n, uint8_t *out);

}  // namespace rie
