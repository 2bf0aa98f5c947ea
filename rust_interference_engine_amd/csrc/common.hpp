// common.hpp — shared definitions of the rie-hip runtime (host and device).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace rie {

// ggml type ids (quant/mod.rs:34-51 in the reference)
enum GgmlType : int {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8,
    T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_BF16 = 30
};

// Error codes of the C ABI: one per variant of the reference's Error enum
// (error.rs:5-15), negative.
enum ErrCode : int { E_OK = 0, E_IO = -1, E_FORMAT = -2, E_UNSUPPORTED = -3, E_MISSING = -4, E_RUNTIME = -5 };

struct Error {
    int code;
    std::string msg;
};

inline size_t block_size(int ty) {
    switch (ty) {
    case T_F32: case T_F16: case T_BF16: return 1;
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: return 32;
    default: return 256;
    }
}

inline size_t block_bytes(int ty) {
    switch (ty) {
    case T_F32: return 4;
    case T_F16: case T_BF16: return 2;
    case T_Q4_0: return 18;
    case T_Q4_1: return 20;
    case T_Q5_0: return 22;
    case T_Q5_1: return 24;
    case T_Q8_0: return 34;
    case T_Q2_K: return 84;
    case T_Q3_K: return 110;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    default: return 0;
    }
}

inline size_t row_bytes(int ty, size_t n) { return n / block_size(ty) * block_bytes(ty); }

inline const char *type_name(int ty) {
    switch (ty) {
    case T_F32: return "F32";
    case T_F16: return "F16";
    case T_BF16: return "BF16";
    case T_Q4_0: return "Q4_0";
    case T_Q4_1: return "Q4_1";
    case T_Q5_0: return "Q5_0";
    case T_Q5_1: return "Q5_1";
    case T_Q8_0: return "Q8_0";
    case T_Q2_K: return "Q2_K";
    case T_Q3_K: return "Q3_K";
    case T_Q4_K: return "Q4_K";
    case T_Q5_K: return "Q5_K";
    case T_Q6_K: return "Q6_K";
    default: return "?";
    }
}

// Activation formats a weight type consumes (quant/mod.rs:118-124).
enum ActFmt : int { ACT_F32 = 0, ACT_Q8_0 = 1, ACT_Q8K = 2 };

inline int act_format(int ty) {
    switch (ty) {
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: return ACT_Q8_0;
    case T_Q4_K: case T_Q5_K: case T_Q6_K: case T_Q2_K: case T_Q3_K: return ACT_Q8K;
    default: return ACT_F32;
    }
}

// Device layout of a quantized activation batch (n rows of k values).
// Q8_0 (32-blocks):  qs int8 [n][k], d f32 [n][k/32], s f32 [n][k/32] (= d·Σ unclamped
//                    codes, the reference BlockQ8_0::s), isum i32 [n][k/32] (Σ clamped codes)
// Q8_K (256-blocks): qs int8 [n][k], d f32 [n][k/256], bsums i16 [n][k/16]
struct ActQ8 {
    int8_t *qs = nullptr;
    float *d = nullptr;
    float *s = nullptr;
    int32_t *isum = nullptr;
    int16_t *bsums = nullptr;
};

// A weight matrix resident in HBM in its native ggml block layout.
struct DevWeight {
    int ty = -1;
    size_t rows = 0, cols = 0;
    const uint8_t *data = nullptr;  // device pointer, row r at data + r*row_bytes(ty, cols)
    size_t rb() const { return row_bytes(ty, cols); }
};

}  // namespace rie

#define RIE_HIP_CHECK(expr)                                                                    \
    do {                                                                                       \
        hipError_t e_ = (expr);                                                                \
        if (e_ != hipSuccess)                                                                  \
            throw rie::Error{rie::E_RUNTIME, std::string("HIP error ") + hipGetErrorString(e_) + \
                                                 " at " + __FILE__ + ":" + std::to_string(__LINE__)}; \
    } while (0)
