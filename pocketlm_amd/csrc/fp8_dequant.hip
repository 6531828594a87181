// FP8 e4m3 block-scaled dequant (src/pcketlm/native/fp8_dequant.cpp and the
// fp32 torch branch of fp8_source.py:852-858), bit-exact.
//
// out[r, c] = cvt(dec(W[r, c]) * scale[r/128, c/128]).  The fp32 product is
// formed first.  NaN bytes decode to NaN with payload 0x7FF00000/0xFFF00000
// (fp8_dequant.cpp:22-27) and the product follows x86 SSE rules, which is what
// the reference (and torch on the CPU) computes: a NaN first operand is
// returned quieted, else a NaN second operand, else an invalid product
// (inf * 0) is the x86 default NaN 0xFFC00000.  fp16 rounding is F16C's
// (RNE, NaN -> sign|0x7E00|payload>>13); bf16 is bits + 0x7FFF + lsb with
// every NaN -> 0xFFFF (fp8_dequant.cpp:108-117).
//
// Streaming kernel, HBM-bound on the writes (2 or 4 bytes per weight byte):
// every wave-wide store is 1 KB contiguous.
#include "common.h"

namespace {

constexpr int kSegCols = 8192;  // columns of one row per workgroup

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

__device__ __forceinline__ bool is_nan_bits(uint32_t b) { return (b & 0x7FFFFFFFu) > 0x7F800000u; }

// x86 mulss/mulps result bits for a * b.
__device__ __forceinline__ uint32_t x86_mul_bits(float a, float b) {
    const uint32_t ab = f2u(a), bb = f2u(b);
    if (is_nan_bits(ab)) return ab | 0x00400000u;
    if (is_nan_bits(bb)) return bb | 0x00400000u;
    const float r = a * b;
    return r != r ? 0xFFC00000u : f2u(r);
}

// F16C vcvtps2ph with round-to-nearest-even.
__device__ __forceinline__ uint16_t f16_bits_f16c(uint32_t bits) {
    if (is_nan_bits(bits)) {
        return static_cast<uint16_t>(((bits >> 16) & 0x8000u) | 0x7E00u | ((bits & 0x7FFFFFu) >> 13));
    }
    const _Float16 h = static_cast<_Float16>(u2f(bits));
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ uint16_t bf16_bits(uint32_t bits) {
    if (is_nan_bits(bits)) return 0xFFFFu;
    return static_cast<uint16_t>((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

// Hardware decode with the dequant NaN payload.
__device__ __forceinline__ void decode4_dequant(uint32_t d, float* v) {
    plm_decode4_e4m3(d, v);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t byte = (d >> (8 * j)) & 0xFFu;
        if ((byte & 0x7Fu) == 0x7Fu) v[j] = u2f((byte & 0x80u) ? 0xFFF00000u : 0x7FF00000u);
    }
}

// True when one of the four bytes of d is an e4m3 NaN (0x7F / 0xFF).
__device__ __forceinline__ bool has_nan_byte(uint32_t d) {
    return (((d & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u) != 0u;
}

template <int OUT>
__device__ __forceinline__ uint32_t out_bits16(uint32_t bits) {
    return OUT == 0 ? f16_bits_f16c(bits) : bf16_bits(bits);
}

// Dequantize the 4 bytes of d with scale sc into 4 fp32 bit patterns.
__device__ __forceinline__ void deq4(uint32_t d, float sc, bool exact, uint32_t* bits) {
    float v[4];
    if (exact) {
        decode4_dequant(d, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) bits[j] = x86_mul_bits(v[j], sc);
    } else {
        plm_decode4_e4m3(d, v);
#pragma unroll
        for (int j = 0; j < 4; ++j) bits[j] = f2u(v[j] * sc);
    }
}

// One workgroup covers kSegCols columns of one row.  For 16-bit outputs a lane
// reads 8 bytes and writes 16 per pass, for fp32 it reads 4 and writes 16,
// so every wave-wide store is 1 KB contiguous.  All passes' loads are issued
// first (addresses past the row end are clamped and their results dropped),
// so a workgroup waits for memory once.  Finite spans take the plain
// multiply; spans holding a NaN byte (or a non-finite scale) take the exact
// x86 emulation.
template <int OUT>
__global__ __launch_bounds__(256) void fp8_dequant_kernel(const uint8_t* __restrict__ w, const float* __restrict__ s,
                                                          void* __restrict__ out, int64_t cols, int64_t scale_cols,
                                                          int segs_per_row) {
    constexpr int BPL = OUT == 2 ? 4 : 8;          // input bytes per lane per pass
    constexpr int PASSES = kSegCols / (256 * BPL);  // 8 (fp32) or 4 (16-bit)
    const int64_t row = blockIdx.x / segs_per_row;
    const int seg = blockIdx.x - static_cast<int>(row) * segs_per_row;
    const float* srow = s + (row >> 7) * scale_cols;
    int64_t col[PASSES];
    uint2 d[PASSES];
    float sc[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        col[p] = static_cast<int64_t>(seg) * kSegCols + (p * 256 + threadIdx.x) * BPL;
        const int64_t cc = col[p] < cols ? col[p] : cols - BPL;
        if constexpr (OUT == 2) {
            d[p].x = *reinterpret_cast<const uint32_t*>(w + row * cols + cc);
        } else {
            d[p] = *reinterpret_cast<const uint2*>(w + row * cols + cc);
        }
        sc[p] = srow[cc >> 7];
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        if (col[p] >= cols) break;
        const int64_t idx = row * cols + col[p];
        const bool sc_finite = (f2u(sc[p]) & 0x7F800000u) != 0x7F800000u;
        if constexpr (OUT == 2) {
            uint32_t b[4];
            deq4(d[p].x, sc[p], !sc_finite || has_nan_byte(d[p].x), b);
            *reinterpret_cast<uint4*>(static_cast<float*>(out) + idx) = make_uint4(b[0], b[1], b[2], b[3]);
        } else {
            const bool exact = !sc_finite || has_nan_byte(d[p].x) || has_nan_byte(d[p].y);
            uint32_t b[8];
            deq4(d[p].x, sc[p], exact, b);
            deq4(d[p].y, sc[p], exact, b + 4);
            uint32_t h[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) h[i] = out_bits16<OUT>(b[2 * i]) | (out_bits16<OUT>(b[2 * i + 1]) << 16);
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + idx) = make_uint4(h[0], h[1], h[2], h[3]);
        }
    }
}

template <int OUT>
__global__ void fp8_dequant_scalar_kernel(const uint8_t* w, const float* s, void* out, int64_t rows, int64_t cols,
                                          int64_t scale_cols) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= rows * cols) return;
    const int64_t row = idx / cols;
    const int64_t col = idx - row * cols;
    float v[4];
    decode4_dequant(w[idx], v);
    const uint32_t b = x86_mul_bits(v[0], s[(row >> 7) * scale_cols + (col >> 7)]);
    if constexpr (OUT == 2) {
        static_cast<float*>(out)[idx] = u2f(b);
    } else {
        static_cast<uint16_t*>(out)[idx] = OUT == 0 ? f16_bits_f16c(b) : bf16_bits(b);
    }
}

template <int OUT>
int dequant(const uint8_t* w, const float* s, void* out, int64_t rows, int64_t cols, int64_t scale_cols) {
    if (!w || !s || !out) return plm::fail(-1, "null pointer");
    if (rows <= 0 || cols <= 0 || scale_cols <= 0) return plm::fail(-2, "bad dimensions");
    if (scale_cols != plm::ceil_div(cols, 128)) return plm::fail(-3, "scale_cols != ceil(cols/128)");
    hipStream_t st = plm::current_stream();
    if (cols % 16 == 0 && plm::aligned16(w) && plm::aligned16(out)) {
        const int64_t segs = plm::ceil_div(cols, kSegCols);
        const int64_t grid = rows * segs;
        if (grid > 0x7FFFFFFF) return plm::fail(-2, "tensor too large");
        hipLaunchKernelGGL((fp8_dequant_kernel<OUT>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, st, w, s, out,
                           cols, scale_cols, static_cast<int>(segs));
    } else {
        const int64_t blocks = plm::ceil_div(rows * cols, 256);
        hipLaunchKernelGGL((fp8_dequant_scalar_kernel<OUT>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                           w, s, out, rows, cols, scale_cols);
    }
    return plm::check_launch("fp8 dequant kernel");
}

}  // namespace

PLM_EXPORT int fp8_e4m3_dequant_to_fp16(const uint8_t* fp8_weight, const float* scale_inv, uint16_t* out_fp16,
                                        int64_t rows, int64_t cols, int64_t scale_cols) {
    return dequant<0>(fp8_weight, scale_inv, out_fp16, rows, cols, scale_cols);
}

PLM_EXPORT int fp8_e4m3_dequant_to_bf16(const uint8_t* fp8_weight, const float* scale_inv, uint16_t* out_bf16,
                                        int64_t rows, int64_t cols, int64_t scale_cols) {
    return dequant<1>(fp8_weight, scale_inv, out_bf16, rows, cols, scale_cols);
}

PLM_EXPORT int fp8_e4m3_dequant_to_f32(const uint8_t* fp8_weight, const float* scale_inv, float* out_f32,
                                       int64_t rows, int64_t cols, int64_t scale_cols) {
    return dequant<2>(fp8_weight, scale_inv, out_f32, rows, cols, scale_cols);
}
