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
//   * topk_level_kernel: slices of 1024 entries, one wave each, keep their
//     top_k (a larger value first, equal values by the lower row), found by
//     a bisection on order-preserving keys counted with ballots; levels
//     repeat on the survivors until one slice writes the top_k in
//     descending order (top_k <= 64).  NaN logits rank as -inf.  With fewer
//     rows than top_k the remaining slots are id -1, logit -inf, the
//     reference's initial values.
#include <algorithm>

#include "common.h"

namespace {

constexpr int kLmRowsPerWave = 4;
constexpr int kLmWaves = 4;              // 256 threads: 16 rows per workgroup
constexpr int kTopkJ = 16;               // entries per lane of a selection slice (1024 per slice)
constexpr int kTopkWaves = 4;            // slices per workgroup of a reducing level
constexpr int kTopkFinalWaves = 8;       // slices of the last two levels (one workgroup)
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
// U: 16-byte pieces in flight per lane (a row of up to 64 U pieces in one
// round of loads).
template <bool BF16, int U>
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
        for (int c0 = lane; c0 < nx; c0 += 64 * U) {
            uint4 q[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int c = c0 + u * 64;
                q[u] = wr[c < nx ? c : nx - 1];  // in range; an out-of-range piece is not used
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
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

// LDS writes of a wave made visible to its other lanes.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Set lanes of m below this lane.
__device__ __forceinline__ int lanes_below(unsigned long long m) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

// Top-k selection.  A slice of 64 J entries (J per lane of one wave, entry j
// of lane l at position 64 j + l) keeps its top_k in rank order: a larger
// value first, equal values by position.  The first level's rows rise with
// the position, and every later level stores a slice's survivors in rank
// order, slices in row order, so the lower position is the lower row.  No
// barrier: a 32-step bisection on the order-preserving keys, counted with
// ballots, finds the top_k-th largest key T; entries above T and the
// lowest-placed entries equal to T make exactly top_k survivors (fewer when
// the slice holds fewer), ranked among themselves.  Missing ranks of a level
// that is not the last are (NaN, -1), which the next level reads as absent
// (no kept value is NaN: NaN logits rank as -inf); the last level writes ids
// + token_offset and logits, (-1, -inf) past the available entries.

// Keys of one slice's entries (0: absent).  FIRST: the values are logits.
template <bool FIRST, int J>
__device__ __forceinline__ void slice_keys(float (&val)[J], uint32_t (&key)[J], int64_t avail, int lane) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool ok = j * 64 + lane < avail && (FIRST || val[j] == val[j]);
        val[j] = ok ? (FIRST ? key_of(val[j]) : val[j]) : 0.0f;
        key[j] = ok ? order_key(val[j]) : 0u;
    }
}

// The slice's survivors, unranked, in sv / sp [0, kept) (value, position),
// and entries after them in [kept, 64) that rank after every survivor;
// returns kept.  Every lane of the wave calls it.
template <int J>
__device__ __forceinline__ int slice_survivors(const float (&val)[J], const uint32_t (&key)[J], int top_k, float* sv,
                                               int* sp, int lane) {
    auto count_at_least = [&](uint32_t t) {
        int c = 0;
#pragma unroll
        for (int j = 0; j < J; ++j) c += __popcll(__ballot(key[j] >= t));
        return c;
    };
    // T: the largest t with at least top_k entries at or above it (0 when
    // the slice holds fewer than top_k entries: all of them survive)
    uint32_t T = 0u;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = T | (1u << bit);
        if (count_at_least(cand) >= top_k) T = cand;
    }
    const int need = top_k - (T == 0u ? 0 : count_at_least(T + 1u));  // ties kept, lowest positions first
    int ties = 0, kept = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool tie = key[j] != 0u && key[j] == T;
        const unsigned long long tm = __ballot(tie);
        const bool keep = key[j] != 0u && (key[j] > T || (tie && ties + lanes_below(tm) < need));
        ties += __popcll(tm);
        const unsigned long long km = __ballot(keep);
        if (keep) {
            const int slot = kept + lanes_below(km);
            sv[slot] = val[j];
            sp[slot] = j * 64 + lane;
        }
        kept += __popcll(km);  // at most top_k
    }
    if (lane >= kept) {
        sv[lane] = -__builtin_inff();
        sp[lane] = 0x7FFFFFFF;
    }
    wave_sync();
    return kept;
}

// Rank of survivor (c, pi) among the 64 slots.
__device__ __forceinline__ int survivor_rank(const float* sv, const int* sp, float c, int pi) {
    int rank = 0;
#pragma unroll 4
    for (int j = 0; j < kMaxTopK; j += 4) {
        const float4 v = *reinterpret_cast<const float4*>(sv + j);
        const int4 q = *reinterpret_cast<const int4*>(sp + j);
        rank += (v.x > c) || (v.x == c && q.x < pi);
        rank += (v.y > c) || (v.y == c && q.y < pi);
        rank += (v.z > c) || (v.z == c && q.z < pi);
        rank += (v.w > c) || (v.w == c && q.w < pi);
    }
    return rank;
}

// One reducing level: slice b of in keeps its top_k at out[b * top_k + rank].
template <bool FIRST>
__global__ __launch_bounds__(kTopkWaves * 64) void topk_level_kernel(const float* __restrict__ in_v,
                                                                     const int64_t* __restrict__ in_r, int64_t n_in,
                                                                     int top_k, float* __restrict__ out_v,
                                                                     int64_t* __restrict__ out_r) {
    constexpr int J = kTopkJ;
    __shared__ __align__(16) float sv[kTopkWaves][kMaxTopK];
    __shared__ __align__(16) int sp[kTopkWaves][kMaxTopK];
    const int wave = static_cast<int>(threadIdx.x >> 6);
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int64_t slice = static_cast<int64_t>(blockIdx.x) * kTopkWaves + wave;
    const int64_t base = slice * (64 * J);
    if (base >= n_in) return;  // a whole wave; no barrier below
    // every load issued before the first use (entries past the end read the
    // last one and are dropped)
    float val[J];
    uint32_t key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) val[j] = in_v[min(base + j * 64 + lane, n_in - 1)];
    __builtin_amdgcn_sched_barrier(0);  // keep the loads together
    slice_keys<FIRST, J>(val, key, n_in - base, lane);
    const int kept = slice_survivors<J>(val, key, top_k, sv[wave], sp[wave], lane);
    const int64_t o = slice * top_k;
    if (lane < kept) {
        const float c = sv[wave][lane];
        const int pi = sp[wave][lane];
        const int rank = survivor_rank(sv[wave], sp[wave], c, pi);
        out_v[o + rank] = c;
        out_r[o + rank] = FIRST ? base + pi : in_r[base + pi];
    } else if (lane < top_k) {
        out_v[o + lane] = __builtin_nanf("");
        out_r[o + lane] = -1;
    }
}

// The last two levels in one workgroup: wave w takes slice w of in (at most
// kTopkFinalWaves slices) and leaves its survivors in rank order in LDS;
// then wave 0 selects the top_k of those and writes ids + token_offset and
// logits.
template <bool FIRST>
__global__ __launch_bounds__(kTopkFinalWaves * 64) void topk_final_kernel(const float* __restrict__ in_v,
                                                                          const int64_t* __restrict__ in_r,
                                                                          int64_t n_in, int top_k,
                                                                          float* __restrict__ out_v,
                                                                          int64_t* __restrict__ out_r,
                                                                          int64_t token_offset) {
    constexpr int J = kTopkJ;
    static_assert(kTopkFinalWaves * kMaxTopK <= 64 * J, "the survivors of every slice fit one slice");
    __shared__ __align__(16) float sv[kTopkFinalWaves][kMaxTopK];
    __shared__ __align__(16) int sp[kTopkFinalWaves][kMaxTopK];
    __shared__ float cv[kTopkFinalWaves * kMaxTopK];
    __shared__ int64_t cr[kTopkFinalWaves * kMaxTopK];
    const int wave = static_cast<int>(threadIdx.x >> 6);
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int64_t base = static_cast<int64_t>(wave) * (64 * J);
    const int nslices = static_cast<int>((n_in + 64 * J - 1) / (64 * J));
    if (base < n_in) {  // whole waves
        float val[J];
        uint32_t key[J];
#pragma unroll
        for (int j = 0; j < J; ++j) val[j] = in_v[min(base + j * 64 + lane, n_in - 1)];
        __builtin_amdgcn_sched_barrier(0);
        slice_keys<FIRST, J>(val, key, n_in - base, lane);
        const int kept = slice_survivors<J>(val, key, top_k, sv[wave], sp[wave], lane);
        const int o = wave * top_k;
        if (lane < kept) {
            const float c = sv[wave][lane];
            const int pi = sp[wave][lane];
            const int rank = survivor_rank(sv[wave], sp[wave], c, pi);
            cv[o + rank] = c;
            cr[o + rank] = FIRST ? base + pi : in_r[base + pi];
        } else if (lane < top_k) {
            cv[o + lane] = __builtin_nanf("");
            cr[o + lane] = -1;
        }
    }
    __syncthreads();
    if (wave != 0) return;
    const int n2 = nslices * top_k;
    float val[J];
    uint32_t key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) val[j] = cv[min(j * 64 + lane, n2 - 1)];
    slice_keys<false, J>(val, key, n2, lane);
    const int kept = slice_survivors<J>(val, key, top_k, sv[0], sp[0], lane);
    if (lane < kept) {
        const float c = sv[0][lane];
        const int pi = sp[0][lane];
        const int rank = survivor_rank(sv[0], sp[0], c, pi);
        out_v[rank] = c;
        out_r[rank] = cr[pi] + token_offset;
    } else if (lane < top_k) {
        out_v[lane] = -__builtin_inff();
        out_r[lane] = -1;
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
    // candidates of the first level; later levels are smaller (top_k <= 64 * kTopkJ / 32)
    const int64_t cand_half = plm::ceil_div(plm::ceil_div(rows, 64 * kTopkJ) * top_k, 64) * 64;
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
        // rows of more than 512 pieces in one round of 16 loads per lane (DeepSeek-V3's
        // 7168 columns), shorter rows in rounds of 8
        const bool wide = hidden_size / 8 > 64 * 8;
        auto kern = dtype_code == 1 ? (wide ? lm_head_logits_kernel<true, 16> : lm_head_logits_kernel<true, 8>)
                                    : (wide ? lm_head_logits_kernel<false, 16> : lm_head_logits_kernel<false, 8>);
        hipLaunchKernelGGL(kern, grid, dim3(kLmWaves * 64), shmem, st, hidden, weight, logits, rows, hidden_size);
    } else {
        hipLaunchKernelGGL(lm_head_logits_scalar_kernel, dim3(static_cast<unsigned>(plm::ceil_div(rows, 256))),
                           dim3(256), 0, st, hidden, weight, logits, rows, hidden_size, dtype_code);
    }
    int code = plm::check_launch("lm_head logits kernel");
    if (code != 0) return code;
    // levels of slices keeping their top_k, until one slice is left
    const float* in_v = logits;
    const int64_t* in_r = nullptr;
    int64_t n = rows;
    bool first = true;
    float* bufs_v[2] = {cand_v, cand_v + cand_half};
    int64_t* bufs_r[2] = {cand_r, cand_r + cand_half};
    for (int level = 0;; ++level) {
        const int64_t blocks = plm::ceil_div(n, 64 * kTopkJ);  // slices
        if (blocks <= kTopkFinalWaves) {
            auto kern = first ? topk_final_kernel<true> : topk_final_kernel<false>;
            hipLaunchKernelGGL(kern, dim3(1), dim3(kTopkFinalWaves * 64), 0, st, in_v, in_r, n, static_cast<int>(top_k),
                               out_logits, out_ids, token_offset);
            return plm::check_launch("top-k final kernel");
        }
        float* ov = bufs_v[level & 1];
        int64_t* orow = bufs_r[level & 1];
        auto kern = first ? topk_level_kernel<true> : topk_level_kernel<false>;
        hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(plm::ceil_div(blocks, kTopkWaves))), dim3(kTopkWaves * 64),
                           0, st, in_v, in_r, n, static_cast<int>(top_k), ov, orow);
        code = plm::check_launch("top-k level kernel");
        if (code != 0) return code;
        in_v = ov;
        in_r = orow;
        n = blocks * top_k;
        first = false;
    }
}
