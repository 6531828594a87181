// row8-packed fp16/bf16 GEMV for gfx950 (src/pcketlm/native/fp16_packed_gemv.cpp
// and the fused variants of fp16_kv_cache.cpp:117-298, including the fp32
// activation variant used for the o and down projections, 146-174).
//
// Layout: packed[blk][k][lane] = W[8*blk + lane][k], so one 8-row block is a
// contiguous K x 16-byte run.  A lane loads one 16-byte column slice (the 8
// rows of column k) and does 8 FMAs with x[k]; 64 lanes cover 64 columns = 1 KB
// per wave per chunk.  fp32 accumulation with fused multiply-add, as the
// reference's _mm256_fmadd_ps.
#include <algorithm>
#include <cstring>

#include "row8.h"

namespace {

constexpr int kMaxWaves = 8;
constexpr int kUnroll = 8;       // chunks whose loads are issued together
constexpr int kMaxMats = plm::kRow8MaxMats;  // matrices per fused launch
using plm::Row8Mat;

__device__ __forceinline__ float u16_to_f32(uint32_t v, int bf16) {
    if (bf16) return __uint_as_float(v << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v)));
}

__device__ __forceinline__ void decode8(const uint4& q, int bf16, float* w) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (bf16) {
            w[2 * i] = __uint_as_float(d[i] << 16);
            w[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
        } else {
            w[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(d[i] & 0xFFFFu)));
            w[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(d[i] >> 16)));
        }
    }
}

// Activation source of a launch (template parameter XM).
enum XMode { kXU16 = 0, kXF32 = 1, kXSilu = 2, kXNorm = 3 };

// fp32 -> fp16 (round to nearest even) / bf16 (add 0x7FFF + lsb, truncate).
__device__ __forceinline__ uint16_t f32_to_u16(float v, bool bf16) {
    if (bf16) {
        const uint32_t bits = __float_as_uint(v);
        return static_cast<uint16_t>((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
    }
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

struct Row8Args {
    Row8Mat mat[kMaxMats];
    const uint16_t* hidden;      // fp16 / bf16 activations (same type as the weights), or
    const float* hidden_f32;     // fp32 activations
    const float* hidden_b;       // kXSilu: the up values
    const uint16_t* norm_w;      // kXNorm: the norm weight
    float eps;
    int64_t K;
    int nmats;
    int nchunks;           // ceil(K / 64)
    int bf16;
};

// One workgroup = one 8-row block of one matrix; its waves split the columns.
template <bool BF16, int XM>
__global__ __launch_bounds__(512) void row8_gemv_kernel(const Row8Args a) {
#pragma clang fp contract(off)
    __shared__ float red[kMaxWaves * 8];
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    int mi = 0;
#pragma unroll 1
    for (int i = 1; i < a.nmats; ++i)
        if (static_cast<int64_t>(blockIdx.x) >= a.mat[i].first_tile) mi = i;
    const Row8Mat m = a.mat[mi];
    const int64_t blk = blockIdx.x - m.first_tile;
    const uint16_t* base = m.packed + blk * a.K * 8;

    float scale = 1.0f;
    if (XM == kXNorm) {  // every workgroup reduces the (small) hidden vector itself
        float ss = 0.0f;
        for (int64_t i = threadIdx.x; i < a.K; i += blockDim.x) {
            const float v = u16_to_f32(a.hidden[i], BF16);
            ss += v * v;
        }
        const float t = plm_wave_sum(ss);
        if (lane == kSumLane) red[wave] = t;
        __syncthreads();
        ss = 0.0f;
        for (int w = 0; w < nw; ++w) ss += red[w];
        scale = 1.0f / sqrtf(ss / static_cast<float>(a.K) + a.eps);
        __syncthreads();
    }

    float acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = 0.0f;

    for (int c0 = wave; c0 < a.nchunks; c0 += nw * kUnroll) {
        uint4 q[kUnroll];
        float xv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            // Unconditional loads from a clamped column (its x is zeroed) so
            // that every load of the group issues before the first wait.
            const int64_t col = static_cast<int64_t>(c0 + u * nw) * 64 + lane;
            const bool ok = c0 + u * nw < a.nchunks && col < a.K;
            const int64_t cc = ok ? col : a.K - 1;
            q[u] = *reinterpret_cast<const uint4*>(base + cc * 8);
            float xh;
            if (XM == kXU16) {
                xh = u16_to_f32(a.hidden[cc], BF16);
            } else if (XM == kXF32) {
                xh = a.hidden_f32[cc];
            } else if (XM == kXSilu) {
                const float g = a.hidden_f32[cc];
                xh = (g / (1.0f + expf(-g))) * a.hidden_b[cc];
            } else {
                const float n = u16_to_f32(a.hidden[cc], BF16) * scale * u16_to_f32(a.norm_w[cc], BF16);
                xh = u16_to_f32(f32_to_u16(n, BF16), BF16);
            }
            xv[u] = ok ? xh : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            float w[8];
            decode8(q[u], BF16, w);
#pragma unroll
            for (int l = 0; l < 8; ++l) acc[l] = fmaf(xv[u], w[l], acc[l]);
        }
    }
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        const float t = plm_wave_sum(acc[l]);
        if (lane == kSumLane) red[wave * 8 + l] = t;
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        const int l = threadIdx.x;
        const int64_t row = blk * 8 + l;
        if (row < m.rows) {
            float v = 0.0f;
            for (int w = 0; w < nw; ++w) v += red[w * 8 + l];
            if (m.bias) v += u16_to_f32(m.bias[row], BF16);
            if (m.out16) {
                m.out16[row] = f32_to_u16(m.resid[row] + v, BF16);
            } else {
                m.out[row] = v;
            }
        }
    }
}

// Pack: one thread per (block, column) writes the 16-byte column slice.
__global__ void pack_rows8_kernel(const uint16_t* __restrict__ w, uint16_t* __restrict__ packed, int64_t rows,
                                  int64_t cols) {
    const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t blocks = (rows + 7) / 8;
    if (id >= blocks * cols) return;
    const int64_t blk = id / cols;
    const int64_t col = id - blk * cols;
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t r0 = blk * 8 + 2 * i, r1 = r0 + 1;
        const uint32_t lo = r0 < rows ? w[r0 * cols + col] : 0u;
        const uint32_t hi = r1 < rows ? w[r1 * cols + col] : 0u;
        h[i] = lo | (hi << 16);
    }
    uint16_t* dst = packed + id * 8;
    if ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(h[0], h[1], h[2], h[3]);
    } else {
        for (int i = 0; i < 4; ++i) {
            dst[2 * i] = static_cast<uint16_t>(h[i] & 0xFFFFu);
            dst[2 * i + 1] = static_cast<uint16_t>(h[i] >> 16);
        }
    }
}

int run_row8(const plm::Row8X& x, const Row8Mat* mats, int n, int64_t K, int dtype_code, hipStream_t st) {
    Row8Args a;
    std::memset(&a, 0, sizeof(a));
    int64_t tiles = 0;
    int used = 0;
    for (int i = 0; i < n; ++i) {
        if (mats[i].rows <= 0) continue;
        if (!plm::aligned16(mats[i].packed)) return plm::fail(2, "packed weight not 16-byte aligned");
        a.mat[used] = mats[i];
        a.mat[used].first_tile = tiles;
        tiles += (mats[i].rows + 7) / 8;
        ++used;
    }
    if (used == 0) return 0;  // nothing to write
    a.hidden = x.u16;
    a.hidden_f32 = x.f32;
    a.hidden_b = x.f32_b;
    a.norm_w = x.norm_w;
    a.eps = x.eps;
    a.K = K;
    a.nmats = used;
    a.nchunks = static_cast<int>(plm::ceil_div(K, 64));
    a.bf16 = dtype_code;
    const int nw = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(a.nchunks, kMaxWaves)));
    if (tiles > 0x7FFFFFFF) return plm::fail(2, "too many row blocks");
    const dim3 grid(static_cast<unsigned>(tiles)), block(nw * plm::kWave);
    const int xm = x.f32 != nullptr ? (x.f32_b != nullptr ? kXSilu : kXF32) : (x.norm_w != nullptr ? kXNorm : kXU16);
    auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, st, a); };
    if (dtype_code == 1) {
        if (xm == kXU16) launch(row8_gemv_kernel<true, kXU16>);
        else if (xm == kXF32) launch(row8_gemv_kernel<true, kXF32>);
        else if (xm == kXSilu) launch(row8_gemv_kernel<true, kXSilu>);
        else launch(row8_gemv_kernel<true, kXNorm>);
    } else {
        if (xm == kXU16) launch(row8_gemv_kernel<false, kXU16>);
        else if (xm == kXF32) launch(row8_gemv_kernel<false, kXF32>);
        else if (xm == kXSilu) launch(row8_gemv_kernel<false, kXSilu>);
        else launch(row8_gemv_kernel<false, kXNorm>);
    }
    return plm::check_launch("row8 gemv kernel");
}

}  // namespace

int plm::row8_gemv(const uint16_t* hidden, const float* hidden_f32, const Row8Mat* mats, int n, int64_t K,
                   int dtype_code, hipStream_t st) {
    plm::Row8X x;
    x.u16 = hidden_f32 == nullptr ? hidden : nullptr;
    x.f32 = hidden_f32;
    return run_row8(x, mats, n, K, dtype_code, st);
}

int plm::row8_gemv_x(const Row8X& x, const Row8Mat* mats, int n, int64_t K, int dtype_code, hipStream_t st) {
    return run_row8(x, mats, n, K, dtype_code, st);
}

PLM_EXPORT int native_pack_u16_rows8(const uint16_t* weight, uint16_t* packed, int64_t rows, int64_t cols) {
    if (!weight || !packed) return plm::fail(1, "null pointer");
    if (rows < 0 || cols < 0) return plm::fail(2, "negative dimensions");
    const int64_t total = ((rows + 7) / 8) * cols;
    if (total == 0) return 0;
    hipLaunchKernelGGL(pack_rows8_kernel, dim3(static_cast<unsigned>(plm::ceil_div(total, 256))), dim3(256), 0,
                       plm::current_stream(), weight, packed, rows, cols);
    return plm::check_launch("row8 pack kernel");
}

PLM_EXPORT int native_packed_gemv_rows8(const uint16_t* hidden, const uint16_t* packed, float* out, int64_t rows,
                                        int64_t cols, int dtype_code) {
    if (!hidden || !packed || !out) return plm::fail(1, "null pointer");
    if (rows < 0 || cols < 0 || (dtype_code != 0 && dtype_code != 1)) return plm::fail(2, "bad dimensions or dtype");
    Row8Mat m;
    m.packed = packed;
    m.bias = nullptr;
    m.out = out;
    m.rows = rows;
    m.first_tile = 0;
    return plm::row8_gemv(hidden, nullptr, &m, 1, cols, dtype_code, plm::current_stream());
}

PLM_EXPORT int native_packed_gemv_rows8_many(const uint16_t* hidden, const uint16_t* const* packed_ptrs,
                                             const uint16_t* const* bias_ptrs, float* const* out_ptrs,
                                             const int64_t* rows, int64_t count, int64_t cols, int dtype_code) {
    if (!hidden || !packed_ptrs || !out_ptrs || !rows) return plm::fail(1, "null pointer");
    if (count <= 0 || count > kMaxMats || cols < 0 || (dtype_code != 0 && dtype_code != 1))
        return plm::fail(2, "bad dimensions or dtype");
    Row8Mat mats[kMaxMats];
    for (int64_t i = 0; i < count; ++i) {
        if (!packed_ptrs[i] || !out_ptrs[i] || rows[i] < 0) return plm::fail(1, "null matrix pointer");
        mats[i].packed = packed_ptrs[i];
        mats[i].bias = bias_ptrs ? bias_ptrs[i] : nullptr;
        mats[i].out = out_ptrs[i];
        mats[i].rows = rows[i];
        mats[i].first_tile = 0;
    }
    return plm::row8_gemv(hidden, nullptr, mats, static_cast<int>(count), cols, dtype_code, plm::current_stream());
}

PLM_EXPORT int native_packed_gemv_rows8_f32_hidden(const float* hidden, const uint16_t* packed, float* out, int64_t rows,
                                                   int64_t cols, int dtype_code) {
    if (!hidden || !packed || !out) return plm::fail(1, "null pointer");
    if (rows < 0 || cols < 0 || (dtype_code != 0 && dtype_code != 1)) return plm::fail(2, "bad dimensions or dtype");
    Row8Mat m;
    m.packed = packed;
    m.bias = nullptr;
    m.out = out;
    m.rows = rows;
    m.first_tile = 0;
    return plm::row8_gemv(nullptr, hidden, &m, 1, cols, dtype_code, plm::current_stream());
}
