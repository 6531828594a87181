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
    int64_t first_tile = 0;    // filled in by row8_gemv
    // Epilogue: when out16 is set, out16[row] = storage(resid[row] + y[row])
    // (rounded as the reference's write_u16) and `out` is not written.
    const float* resid = nullptr;
    uint16_t* out16 = nullptr;
};

// The activation vector of a row8 launch (one of):
//   u16            fp16/bf16 values;
//   u16 + norm_w   storage(u16 * (1 / sqrt(mean(u16^2) + eps)) * norm_w), the
//                  reference's rms_norm_one rounded to the storage type;
//   f32            fp32 values;
//   f32 + f32_b    f32 / (1 + exp(-f32)) * f32_b (SiLU(gate) * up).
struct Row8X {
    const uint16_t* u16 = nullptr;
    const uint16_t* norm_w = nullptr;
    float eps = 0.0f;
    const float* f32 = nullptr;
    const float* f32_b = nullptr;
};

constexpr int kRow8MaxMats = 8;

// out_i = W_i x (+ bias_i) for up to kRow8MaxMats matrices sharing x, in one
// launch on `st`.  x is fp16/bf16 (hidden) or fp32 (hidden_f32, hidden null).
int row8_gemv(const uint16_t* hidden, const float* hidden_f32, const Row8Mat* mats, int n, int64_t K, int dtype_code,
              hipStream_t st);
int row8_gemv_x(const Row8X& x, const Row8Mat* mats, int n, int64_t K, int dtype_code, hipStream_t st);

}  // namespace plm
