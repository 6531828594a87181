// lm_head top-k (src/pcketlm/native/fp16_matmul.cpp:136-204): the logits of
// one fp16/bf16 hidden vector against every row of a [rows, hidden] u16
// weight, and the top_k of them with their row ids (+ token_offset); and the
// same file's fp16 matmul (native_fp16_matmul, 344-396).
//
// The weight is the largest single read of a decode step (vocab x hidden, a
// GB or two), so the GEMV streams it once at HBM rate:
//   * lm_head_logits_kernel: a wave owns 4 rows; its lanes read 16-byte
//     pieces of a row (8 values), eight pieces in flight per lane, and fma
//     them in fp32 against the hidden vector staged once per workgroup in
//     LDS; a DPP wave sum ends each row.
//   * topk_level_kernel: blocks of 1024 entries keep their top_k (a larger
//     value first, equal values by the lower row), found by a bisection on
//     order-preserving keys; levels repeat on the survivors until one block
//     writes the top_k in descending order (top_k <= 64).  NaN logits rank
//     as -inf.  With fewer rows than
//     top_k the remaining slots are id -1, logit -inf, the reference's
//     initial values.
#include <algorithm>

#include "common.h"

namespace {

constexpr int kLmRowsPerWave = 4;
constexpr int kLmWaves = 4;              // 256 threads: 16 rows per workgroup
constexpr int kLmUnroll = 8;             // 16-byte pieces in flight per lane
constexpr int kTopkSlice = 1024;         // entries per block of a selection level (one per thread)
constexpr int kTopkThreads = 1024;
constexpr int kMaxTopK = 64;

__device__ __forceinline__ float u16f(uint32_t v, bool bf16) {
    return bf16 ? __uint_as_float(v << 16) : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v)));
}

template <bool BF16>
__device__ __forceinline__ float dot8(const uint4& w, const uint4& x, float acc) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const uint32_t xd[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = fmaf(u16f(wd[i] & 0xFFFFu, BF16), u16f(xd[i] & 0xFFFFu, BF16), acc);
        acc = fmaf(u16f(wd[i] >> 16, BF16), u16f(xd[i] >> 16, BF16), acc);
    }
    return acc;
}

// K % 8 == 0, x and w 16-byte aligned.  Dynamic LDS: K u16 values.
template <bool BF16>
__global__ __launch_bounds__(kLmWaves * 64) void lm_head_logits_kernel(const uint16_t* __restrict__ x,
                                                                       const uint16_t* __restrict__ w,
                                                                       float* __restrict__ logits, int64_t rows,
                                                                       int64_t K) {
    extern __shared__ uint4 xs[];
    const int nx = static_cast<int>(K / 8);
    for (int i = threadIdx.x; i < nx; i += blockDim.x) xs[i] = reinterpret_cast<const uint4*>(x)[i];
    __syncthreads();
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t first = (static_cast<int64_t>(blockIdx.x) * kLmWaves + wave) * kLmRowsPerWave;
    for (int rr = 0; rr < kLmRowsPerWave; ++rr) {
        const int64_t row = first + rr;
        if (row >= rows) break;  // wave-uniform
        const uint4* wr = reinterpret_cast<const uint4*>(w + row * K);
        float acc = 0.0f;
        for (int c0 = lane; c0 < nx; c0 += 64 * kLmUnroll) {
            uint4 q[kLmUnroll];
#pragma unroll
            for (int u = 0; u < kLmUnroll; ++u) {
                const int c = c0 + u * 64;
                q[u] = wr[c < nx ? c : nx - 1];  // in range; an out-of-range piece is not used
            }
#pragma unroll
            for (int u = 0; u < kLmUnroll; ++u) {
                const int c = c0 + u * 64;
                if (c < nx) acc = dot8<BF16>(q[u], xs[c], acc);
            }
        }
        const float t = plm_wave_sum(acc);
        if (lane == kSumLane) logits[row] = t;
    }
}

// Any K or alignment: one thread per row, sequential in k.
__global__ void lm_head_logits_scalar_kernel(const uint16_t* x, const uint16_t* w, float* logits, int64_t rows,
                                             int64_t K, int bf16) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    float acc = 0.0f;
    for (int64_t k = 0; k < K; ++k) acc = fmaf(u16f(w[row * K + k], bf16 != 0), u16f(x[k], bf16 != 0), acc);
    logits[row] = acc;
}

// Ordering key: NaN as -inf.  a ranks before b when a.v > b.v, or equal
// values and a lower row.
__device__ __forceinline__ float key_of(float v) { return v != v ? -__builtin_inff() : v; }

__device__ __forceinline__ bool beats(float va, int64_t ra, float vb, int64_t rb) {
    return va > vb || (va == vb && ra < rb);
}

// Order-preserving key of a non-NaN float; 0 marks a missing entry (every
// float, -inf included, maps above it).
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Entries of the block whose key is at least t (block-wide, every thread
// gets the count).
__device__ __forceinline__ int count_at_least(uint32_t key, uint32_t t, int* wave_cnt) {
    const int wave = threadIdx.x >> 6;
    const unsigned long long m = __ballot(key != 0u && key >= t);
    if ((threadIdx.x & 63) == 0) wave_cnt[wave] = __popcll(m);
    __syncthreads();
    int c = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) c += wave_cnt[w];
    __syncthreads();
    return c;
}

// Exclusive count of set flags at lower positions (block-wide prefix).
__device__ __forceinline__ int prefix_count(bool flag, int* wave_cnt) {
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const unsigned long long m = __ballot(flag);
    if (lane == 0) wave_cnt[wave] = __popcll(m);
    __syncthreads();
    int c = __popcll(m & ((1ull << lane) - 1ull));
    for (int w = 0; w < wave; ++w) c += wave_cnt[w];
    __syncthreads();
    return c;
}

// One selection level: block b takes entries [b * kTopkSlice, ...) of
// (value, row) pairs (first level: the logits, row = index), one per
// thread, and keeps its top_k in rank order at out[b * top_k + rank];
// missing ranks get (-inf, -1).  With final set (one block), writes ids +
// token_offset and logits instead, -1 / -inf past the available entries.
//
// Rank order: a larger value first, equal values by position in the block.
// The first level's rows rise with the position, and every later level
// stores a block's survivors in rank order, blocks in row order, so the
// lower position is the lower row.  The block finds the top_k without
// comparing all pairs: a 32-step bisection on the order-preserving keys
// finds the top_k-th largest key T; entries above T and the lowest-placed
// entries equal to T make exactly top_k survivors, ranked among themselves.
template <bool FIRST>
__global__ __launch_bounds__(kTopkThreads) void topk_level_kernel(const float* __restrict__ in_v,
                                                                  const int64_t* __restrict__ in_r, int64_t n_in,
                                                                  int top_k, float* __restrict__ out_v,
                                                                  int64_t* __restrict__ out_r, int final,
                                                                  int64_t token_offset) {
    static_assert(kTopkSlice == kTopkThreads, "one entry per thread");
    __shared__ int wave_cnt[kTopkThreads / 64];
    __shared__ float sv[kMaxTopK];
    __shared__ int sp[kMaxTopK];
    const int i = threadIdx.x;
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kTopkSlice;
    const int64_t gi = base + i;
    float val = 0.0f;
    uint32_t key = 0u;
    if (gi < n_in && (FIRST || in_r[gi] >= 0)) {
        val = FIRST ? key_of(in_v[gi]) : in_v[gi];
        key = order_key(val);
    }
    const int64_t o = final ? 0 : static_cast<int64_t>(blockIdx.x) * top_k;
    for (int t = i; t < top_k; t += blockDim.x) {
        out_v[o + t] = -__builtin_inff();
        out_r[o + t] = -1;
    }
    // T: the largest t with at least top_k entries at or above it (0 when
    // the block holds fewer than top_k entries: all of them survive)
    uint32_t T = 0u;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = T | (1u << bit);
        if (count_at_least(key, cand, wave_cnt) >= top_k) T = cand;
    }
    const int above = T == 0u ? 0 : count_at_least(key, T + 1u, wave_cnt);
    const bool tie = key != 0u && key == T;
    const int tie_pos = prefix_count(tie, wave_cnt);
    const bool keep = key != 0u && (key > T || (tie && tie_pos < top_k - above));
    const int slot = prefix_count(keep, wave_cnt);
    if (keep) {
        sv[slot] = val;
        sp[slot] = i;
    }
    const int kept = count_at_least(keep ? 1u : 0u, 1u, wave_cnt);  // survivors (<= top_k)
    __syncthreads();
    if (i < kept) {
        const float c = sv[i];
        const int pi = sp[i];
        int rank = 0;
        for (int j = 0; j < kept; ++j) rank += (sv[j] > c) || (sv[j] == c && sp[j] < pi);
        const int64_t row = FIRST ? base + pi : in_r[base + pi];
        out_v[o + rank] = c;
        out_r[o + rank] = final ? row + token_offset : row;
    }
}

// C = A @ B in fp16 with fp32 accumulation (fp16_matmul.cpp:344-396: the
// fp16 operands widened to fp32, an sgemm, the product rounded to fp16 to
// nearest even).  One wave per 16 x 16 tile of C on the matrix cores: fp16
// products are exact in fp32, so the result differs from the fp32 product
// only in the order of the fp32 sums.  An operand of the rarely used
// unquantized path, kept simple: elementwise bounds-checked loads.
typedef _Float16 plm_f16x8 __attribute__((ext_vector_type(8)));
typedef float plm_f32x4_mm __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void fp16_matmul_kernel(const uint16_t* __restrict__ a,
                                                          const uint16_t* __restrict__ b, uint16_t* __restrict__ c,
                                                          int64_t m, int64_t n, int64_t k, int64_t tiles_n,
                                                          int64_t tiles) {
    const int64_t tile = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (tile >= tiles) return;  // whole waves; no barrier below
    const int lane = threadIdx.x & 63;
    const int i = lane & 15, q = lane >> 4;
    const int64_t tm = tile / tiles_n, tn = tile - tm * tiles_n;
    const int64_t row = tm * 16 + i;  // A operand: row i, k = 8q .. 8q + 7 of each step
    const int64_t col = tn * 16 + i;  // B operand: column i, the same k
    plm_f32x4_mm acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t k0 = 0; k0 < k; k0 += 32) {
        plm_f16x8 av, bv;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t kk = k0 + 8 * q + e;
            const uint16_t x = row < m && kk < k ? a[row * k + kk] : uint16_t{0};
            const uint16_t y = col < n && kk < k ? b[kk * n + col] : uint16_t{0};
            av[e] = __builtin_bit_cast(_Float16, x);
            bv[e] = __builtin_bit_cast(_Float16, y);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
    }
    // D: column i, rows 4q .. 4q + 3
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = tm * 16 + 4 * q + j;
        if (r < m && col < n) c[r * n + col] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(acc[j]));
    }
}

}  // namespace

// ====================================================================== C ABI

PLM_EXPORT int native_fp16_matmul(const uint16_t* a, const uint16_t* b, uint16_t* c, int64_t m, int64_t n,
                                  int64_t k) {
    if (!a || !b || !c) return plm::fail(1, "null pointer");
    if (m < 0 || n < 0 || k < 0) return plm::fail(2, "bad dimensions");
    if (m == 0 || n == 0) return 0;
    const int64_t tiles_n = plm::ceil_div(n, 16);
    const int64_t tiles = plm::ceil_div(m, 16) * tiles_n;
    if (plm::ceil_div(tiles, 4) > INT32_MAX) return plm::fail(2, "too many tiles");
    hipLaunchKernelGGL(fp16_matmul_kernel, dim3(static_cast<unsigned>(plm::ceil_div(tiles, 4))), dim3(256), 0,
                       plm::current_stream(), a, b, c, m, n, k, tiles_n, tiles);
    return plm::check_launch("fp16 matmul kernel");
}

PLM_EXPORT int native_lm_head_topk_u16(const uint16_t* hidden, const uint16_t* weight, int64_t* out_ids,
                                       float* out_logits, int64_t rows, int64_t hidden_size, int64_t top_k,
                                       int dtype_code, int64_t token_offset) {
    if (!hidden || !weight || !out_ids || !out_logits) return plm::fail(1, "null pointer");
    if (rows <= 0 || hidden_size <= 0 || top_k <= 0 || (dtype_code != 0 && dtype_code != 1))
        return plm::fail(2, "bad dimensions");
    if (top_k > kMaxTopK) return plm::fail(2, "top_k above %d", kMaxTopK);
    if (rows > (int64_t{1} << 40)) return plm::fail(2, "too many rows");
    hipStream_t st = plm::current_stream();
    // candidates of the first level; later levels are smaller (top_k <= kTopkSlice / 16)
    const int64_t cand_half = plm::ceil_div(plm::ceil_div(rows, kTopkSlice) * top_k, 64) * 64;
    const size_t logit_bytes = static_cast<size_t>(plm::ceil_div(rows * 4, 256) * 256);
    const size_t candv_bytes = static_cast<size_t>(2 * cand_half * 4);
    char* ws = static_cast<char*>(plm::workspace(logit_bytes + candv_bytes + static_cast<size_t>(2 * cand_half) * 8));
    if (ws == nullptr) return -3;
    float* logits = reinterpret_cast<float*>(ws);
    float* cand_v = reinterpret_cast<float*>(ws + logit_bytes);
    int64_t* cand_r = reinterpret_cast<int64_t*>(ws + logit_bytes + candv_bytes);
    const bool fast = hidden_size % 8 == 0 && hidden_size * 2 <= 64 * 1024 && plm::aligned16(hidden) &&
                      plm::aligned16(weight);
    if (fast) {
        const int64_t per_block = kLmWaves * kLmRowsPerWave;
        const dim3 grid(static_cast<unsigned>(plm::ceil_div(rows, per_block)));
        const size_t shmem = static_cast<size_t>(hidden_size) * 2;
        if (dtype_code == 1) {
            hipLaunchKernelGGL(lm_head_logits_kernel<true>, grid, dim3(kLmWaves * 64), shmem, st, hidden, weight,
                               logits, rows, hidden_size);
        } else {
            hipLaunchKernelGGL(lm_head_logits_kernel<false>, grid, dim3(kLmWaves * 64), shmem, st, hidden, weight,
                               logits, rows, hidden_size);
        }
    } else {
        hipLaunchKernelGGL(lm_head_logits_scalar_kernel, dim3(static_cast<unsigned>(plm::ceil_div(rows, 256))),
                           dim3(256), 0, st, hidden, weight, logits, rows, hidden_size, dtype_code);
    }
    int code = plm::check_launch("lm_head logits kernel");
    if (code != 0) return code;
    // levels of 1024-entry blocks keeping their top_k, until one block is left
    const float* in_v = logits;
    const int64_t* in_r = nullptr;
    int64_t n = rows;
    bool first = true;
    float* bufs_v[2] = {cand_v, cand_v + cand_half};
    int64_t* bufs_r[2] = {cand_r, cand_r + cand_half};
    for (int level = 0;; ++level) {
        const int64_t blocks = plm::ceil_div(n, kTopkSlice);
        const int final = blocks == 1 ? 1 : 0;
        float* ov = final ? out_logits : bufs_v[level & 1];
        int64_t* orow = final ? out_ids : bufs_r[level & 1];
        if (first) {
            hipLaunchKernelGGL(topk_level_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kTopkThreads), 0,
                               st, in_v, in_r, n, static_cast<int>(top_k), ov, orow, final, token_offset);
        } else {
            hipLaunchKernelGGL(topk_level_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kTopkThreads), 0,
                               st, in_v, in_r, n, static_cast<int>(top_k), ov, orow, final, token_offset);
        }
        code = plm::check_launch("top-k level kernel");
        if (code != 0 || final) return code;
        in_v = ov;
        in_r = orow;
        n = blocks * top_k;
        first = false;
    }
}
