// The device-side Cactus-Quants weight, shared by the projection kernels.
#pragma once

#include <cstring>

#include "nd_internal.h"

struct nd_cq {
    int device = 0;
    size_t out_feat = 0, in_feat = 0, in_padded = 0, group = 0, num_groups = 0;
    size_t row_bytes = 0, per_byte = 0;
    uint8_t bits = 0;
    int n_levels = 0;
    float levels[16] = {};
    float inv_sqrt_group = 1.0f;  // 1 / sqrtf(group), as hadamard.rs:51-52
    uint8_t *packed = nullptr;    // device [out][row_bytes] (+16 bytes slack)
    float *norms = nullptr;       // device [out][num_groups]
    float *lut = nullptr;         // device [256][per_byte] (empty for 3-bit)
    float *lv = nullptr;          // device levels[16]
    // Rows from which a 2-bit / ternary matvec takes the fp4 matrix-core
    // kernel; set once when the weight is created.
    size_t fp4_min_rows = 0;
};

// f16 -> f32, exact: subnormals, infinities and NaN included (math.rs:53-68).
inline float nd_f16_to_f32(uint16_t bits)
{
    const uint32_t sign = uint32_t(bits >> 15) << 31;
    const uint32_t exp = (bits >> 10) & 0x1F;
    const uint32_t mant = bits & 0x3FF;
    if (exp == 0) {
        const float val = float(mant) / float(1u << 24);
        return sign ? -val : val;
    }
    const uint32_t out = exp == 31 ? (sign | 0x7F800000u | (mant << 13))
                                   : (sign | ((exp + 127 - 15) << 23) | (mant << 13));
    float f;
    std::memcpy(&f, &out, 4);
    return f;
}
