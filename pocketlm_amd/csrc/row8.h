// row8-packed GEMV launcher shared by the kernels of row8.hip and the dense
// decode layer of kv_cache.hip.
#pragma once

#include "common.h"

namespace plm {

// One matrix of a fused row8 launch: packed[blk][k][lane] = W[8*blk + lane][k].
struct Row8Mat {
    const uint16_t* packed;
    const uint16_t* bias;  // may be null
    float* out;
    int64_t rows;
    int64_t first_tile;    // filled in by row8_gemv
};

constexpr int kRow8MaxMats = 8;

// out_i = W_i x (+ bias_i) for up to kRow8MaxMats matrices sharing x, in one
// launch on `st`.  x is fp16/bf16 (hidden) or fp32 (hidden_f32, hidden null).
int row8_gemv(const uint16_t* hidden, const float* hidden_f32, const Row8Mat* mats, int n, int64_t K, int dtype_code,
              hipStream_t st);

}  // namespace plm
