// The device-side Cactus-Quants weight, shared by the projection kernels.
#pragma once

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
};
