// DeepSeek multi-head latent attention (MLA) for one decode token, on the
// device: ds_mla_attention_flash_forward (src/pcketlm/native/ds_forward.cpp:
// 517-597) and the attention block around it, ds_attention_block_forward_f32
// (ds_forward.cpp:647-782).
//
// The latent cache is shared by every head (kv_cache [L][R], pe_cache
// [L][rope]), so the attention is computed in the latent space with the key
// part of kv_b absorbed into the query (q_abs[h] = q_nope[h] . Wk[h], R wide)
// and the value part applied after the softmax (out[h] = latent[h] . Wv[h]^T):
//
//   mla_qabs_kernel       q_abs [H][R]: per head a (nope x R) product; waves
//                         split nope, their partial sums added in wave order.
//                         The 4-wide instance (mla_qabs4_kernel) can also
//                         write the block's RoPE'd q_pe in place of
//                         mla_q_split_kernel.
//   mla_split_kernel      flash-decode partials: workgroup (split, 16 heads)
//                         walks its tokens in tiles of 16 rows staged in LDS
//                         (each latent row is read once for 16 heads); the
//                         scores and the weighted rows are 16 x 16 products
//                         on the matrix cores (fp32), with a running max /
//                         sum per head.
//   mla_merge_kernel      rescales the splits to the global max and divides
//                         by the sum (1 / sum, 0 when the sum is not positive,
//                         as the reference does): latent [H][R].
//   mla_value_kernel      the value rows of kv_b applied to the latent, two
//                         rows per wave.
//
// The block: fp32 GEMVs (one wave per row, float4 loads, a fixed DPP sum),
// RMSNorm and RoPE kernels, the new cache row appended after the previous
// rows, then the three MLA kernels and the output projection; every launch
// on the caller's stream.
#include <cmath>
#include <algorithm>
#include <cstring>

#include "common.h"
#include "pocketlm_hip.h"

int plm_ds_session_note_fused_attention(void* handle);

namespace {

constexpr int kThreads = 256;
constexpr int kHeadsPerGroup = 16;  // heads of one split workgroup
constexpr int kTileTokens = 16;     // latent rows staged per step
constexpr int64_t kMaxRank = 1024;  // the split kernel's largest instance: 16 column tiles per wave,
constexpr int64_t kMaxRope = 256;   // 20 chunks of 16 columns per wave
constexpr int kMaxSplits = 64;
constexpr int kQabsWaves = 16;  // waves of the absorbed-query kernel

// ------------------------------------------------------------------ q_abs
// q_abs[h][r] = sum_d q_nope[h][d] * wkv_b[h][d][r]; grid (H, ceil(R / 64)),
// wave w sums d = w, w + 4, ... for the workgroup's 64 columns (one per lane).
__global__ __launch_bounds__(kThreads) void mla_qabs_kernel(const float* __restrict__ q_nope,
                                                           const float* __restrict__ wkv_b, float* __restrict__ q_abs,
                                                           int64_t nope, int64_t R, int64_t v) {
    __shared__ float part[4][64];
    const int64_t h = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t r = static_cast<int64_t>(blockIdx.y) * 64 + lane;
    const float* qh = q_nope + h * nope;
    const float* wh = wkv_b + h * (nope + v) * R;
    float acc = 0.0f;
    if (r < R) {
        for (int64_t d0 = wave; d0 < nope; d0 += 4 * 8) {
            float vals[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) vals[u] = wh[min(d0 + 4 * u, nope - 1) * R + r];
#pragma unroll
            for (int u = 0; u < 8; ++u) acc = fmaf(d0 + 4 * u < nope ? qh[d0 + 4 * u] : 0.0f, vals[u], acc);
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && r < R) q_abs[h * R + r] = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
}

// The same with float4 columns (R % 4 == 0, aligned): grid (H, ceil(R / 256)),
// NW waves; lane l of every wave takes columns 4 l .. 4 l + 3 of the
// workgroup's 256, wave w the rows d = w, w + NW, ... (8 in flight), and the
// waves' sums are added in wave order.
// RoPE on pairs (x0, x1) of each group of `dim` values (ds_forward.cpp:621-645).
__device__ __forceinline__ void rope_pair(const float* in, float* out, int64_t pair, const float* cs, const float* sn) {
    const float x0 = in[2 * pair], x1 = in[2 * pair + 1];
    const float c = cs[pair], s = sn[pair];
    out[2 * pair] = x0 * c - x1 * s;
    out[2 * pair + 1] = x0 * s + x1 * c;
}

// With rope_in set (the attention block, whose q is [H][nope + rope] rows of
// q_stride floats), workgroup (h, 0) also writes head h's q_pe with RoPE
// (an odd rope width unrotated, ds_forward.cpp:628-630), the values of
// mla_q_split_kernel.
template <int NW>
__global__ __launch_bounds__(NW * 64) void mla_qabs4_kernel(const float* __restrict__ q_nope, int64_t q_stride,
                                                           const float* __restrict__ wkv_b, float* __restrict__ q_abs,
                                                           int64_t nope, int64_t R, int64_t v,
                                                           const float* __restrict__ rope_in, float* __restrict__ q_pe,
                                                           const float* __restrict__ cs, const float* __restrict__ sn,
                                                           int64_t rope) {
    __shared__ float4 part[NW][64];
    const int64_t h = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t c = static_cast<int64_t>(blockIdx.y) * 256 + 4 * lane;
    const float* qh = q_nope + h * q_stride;
    if (rope_in != nullptr && blockIdx.y == 0) {
        const float* in = rope_in + h * q_stride;
        float* out = q_pe + h * rope;
        if ((rope & 1) == 0) {
            for (int64_t p = threadIdx.x; p < rope / 2; p += NW * 64) rope_pair(in, out, p, cs, sn);
        } else {
            for (int64_t d = threadIdx.x; d < rope; d += NW * 64) out[d] = in[d];
        }
    }
    const float* wh = wkv_b + h * (nope + v) * R;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (c < R) {
        for (int64_t d0 = wave; d0 < nope; d0 += NW * 8) {
            float4 vals[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                vals[u] = *reinterpret_cast<const float4*>(wh + min(d0 + NW * u, nope - 1) * R + c);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float qd = d0 + NW * u < nope ? qh[d0 + NW * u] : 0.0f;
                acc.x = fmaf(qd, vals[u].x, acc.x);
                acc.y = fmaf(qd, vals[u].y, acc.y);
                acc.z = fmaf(qd, vals[u].z, acc.z);
                acc.w = fmaf(qd, vals[u].w, acc.w);
            }
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && c < R) {
        float4 t = part[0][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const float4 p = part[w][lane];
            t = make_float4(t.x + p.x, t.y + p.y, t.z + p.z, t.w + p.w);
        }
        *reinterpret_cast<float4*>(q_abs + h * R + c) = t;
    }
}

// ------------------------------------------------------------------ split
// Flash-decode partials on the matrix cores, v_mfma_f32_16x16x4_f32 (fp32
// products and sums; A[i][k] in lane i + 16 k, B[k][j] in lane j + 16 k,
// D[i][j] in lane j + 16 (i / 4), register i % 4).  Workgroup (split, 16
// heads), four waves.  A tile of 16 cache rows is staged in LDS as
// [row][RS]: the latent columns padded with zeros to R16 (a multiple of 16),
// then the rope columns padded to P16; rows past the split are zeros.
//
//  scores  S^T[row][head] = sum_c row[c] * qfull[head][c] (qfull = q_abs then
//          q_pe, padded alike).  The K dimension goes in chunks of 16
//          columns, chunk j to wave j % 4; in a chunk, lane group g = lane /
//          16 takes columns 16 j + 4 g .. 16 j + 4 g + 3 over the four steps,
//          so each lane reads one float4 of the row (LDS) and one of the query
//          (registers, loaded once).  The four waves' partial tiles are added
//          in LDS in wave order: every wave then holds the same scores, lane
//          (head l % 16) registers r = rows 4 g + r.
//  softmax running max / sum per head; the rows of a head are spread over
//          4 registers and 4 lane groups (two cross-group shuffles).
//  values  Lat^T[col][head] += sum_row kv[row][col] * p[row][head], column
//          tiles of 16 dealt out to the waves.  Step s takes row 4 g + s in
//          lane group g: register s of the score tile is already the B
//          operand, and the accumulator of lane l is head l % 16's, so the
//          rescale by exp(m_old - m_new) is a per-lane multiply.
// QC: chunks (and staging float4s) per lane at most; NT: column tiles per
// wave at most.
typedef float mla_f32x4 __attribute__((ext_vector_type(4)));

struct SplitShape {
    int64_t R16, P16, K16, RS, nct;
};

__host__ __device__ inline SplitShape split_shape(int64_t R, int64_t rope) {
    SplitShape s;
    s.R16 = (R + 15) & ~int64_t(15);
    s.P16 = (rope + 15) & ~int64_t(15);
    s.K16 = s.R16 + s.P16;
    s.RS = ((s.K16 + 31) & ~int64_t(31)) + 4;  // rows 4 banks apart
    s.nct = s.R16 / 16;
    return s;
}

size_t split_lds_bytes(int64_t R, int64_t rope) {
    return static_cast<size_t>(kTileTokens * split_shape(R, rope).RS + 4 * 64 * 4) * sizeof(float);
}

__device__ __forceinline__ mla_f32x4 mfma_f32(float a, float b, mla_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// op over lanes l, l ^ 16, l ^ 32, l ^ 48, as (lower row, upper row) pairs
// at each step, so all four lanes get the same bits.
template <typename Op>
__device__ __forceinline__ float cross_groups(float v, Op op) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Columns c0 .. c0 + 3 of a padded [latent | rope] row, zeros outside the
// two parts or when !ok.  VEC: R and rope are multiples of 4 and the rows
// 16-byte aligned; the load is always issued, from krow when the columns are
// padding, and masked afterwards (bitwise, so the zeros are exact).
template <bool VEC>
__device__ __forceinline__ float4 padded4(const float* krow, const float* prow, int c0, int R, int R16, int rope,
                                          bool ok) {
    if constexpr (VEC) {
        const bool in_k = c0 < R, in_p = !in_k && c0 >= R16 && c0 < R16 + rope;
        const float* base = in_p ? prow : krow;
        const int off = in_k ? c0 : (in_p ? c0 - R16 : 0);
        const uint4 x = *reinterpret_cast<const uint4*>(base + off);
        const uint32_t m = ok && (in_k || in_p) ? ~0u : 0u;
        return make_float4(__uint_as_float(x.x & m), __uint_as_float(x.y & m), __uint_as_float(x.z & m),
                           __uint_as_float(x.w & m));
    } else {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + i;
            e[i] = !ok ? 0.0f : (c < R ? krow[c] : (c >= R16 && c < R16 + rope ? prow[c - R16] : 0.0f));
        }
        return make_float4(e[0], e[1], e[2], e[3]);
    }
}

template <int QC, int NT, bool VEC>
__global__ __launch_bounds__(kThreads) void mla_split_kernel(const float* __restrict__ q_abs,
                                                            const float* __restrict__ q_pe,
                                                            const float* __restrict__ kv, const float* __restrict__ pe,
                                                            float* __restrict__ part, float* __restrict__ ml,
                                                            int64_t H, int64_t L, int64_t R64, int64_t rope64,
                                                            float scale, int64_t per_split) {
    extern __shared__ float4 sm4[];
    float* tile = reinterpret_cast<float*>(sm4);  // [16][RS]
    const SplitShape sh = split_shape(R64, rope64);
    const int R = static_cast<int>(R64), rope = static_cast<int>(rope64);
    const int R16 = static_cast<int>(sh.R16), K16 = static_cast<int>(sh.K16), RS = static_cast<int>(sh.RS);
    const int nct = R16 / 16;
    mla_f32x4* red = reinterpret_cast<mla_f32x4*>(tile + kTileTokens * RS);  // [4 waves][64 lanes]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hl = lane & 15, g = lane >> 4;
    const int64_t h = static_cast<int64_t>(blockIdx.y) * kHeadsPerGroup + hl;
    const bool live = h < H;
    // the row padding [K16, RS) is zero for good: chunks past K16 read it
    for (int i = tid; i < kTileTokens * (RS - K16); i += kThreads) {
        const int r = i / (RS - K16);
        tile[r * RS + K16 + (i - r * (RS - K16))] = 0.0f;
    }
    const int64_t t_begin = static_cast<int64_t>(blockIdx.x) * per_split;
    const int64_t t_end = min(L, t_begin + per_split);

    // the query chunks of this wave, for head hl (a dead head reads head 0, weighted 0)
    float4 q[QC];
    {
        const int64_t hq = live ? h : 0;
        const float* qrow = q_abs + hq * R;
        const float* prow = q_pe + hq * rope;
#pragma unroll
        for (int jj = 0; jj < QC; ++jj) {
            const int c0 = 16 * (wave + 4 * jj) + 4 * g;
            q[jj] = padded4<VEC>(qrow, prow, c0, R, R16, rope, live);
        }
    }
    // staging: thread (row tid / 16) takes float4 columns tid % 16 + 16 k of the row
    const int sr = tid >> 4, sq = tid & 15;
    float4 st[QC];
    auto fetch = [&](int64_t t0, int n) {
        const int64_t t = t0 + (sr < n ? sr : 0);
        const float* krow = kv + t * R;
        const float* prow = pe + t * rope;
#pragma unroll
        for (int k = 0; k < QC; ++k) st[k] = padded4<VEC>(krow, prow, 4 * sq + 64 * k, R, R16, rope, sr < n);
    };
    mla_f32x4 acc[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) acc[i] = mla_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    int n = static_cast<int>(min(static_cast<int64_t>(kTileTokens), t_end - t_begin));
    fetch(t_begin, n);
    for (int64_t t0 = t_begin; t0 < t_end; t0 += kTileTokens) {
        __syncthreads();  // the previous tile's readers are done
#pragma unroll
        for (int k = 0; k < QC; ++k)  // columns past K16 land in the row's padding
            *reinterpret_cast<float4*>(tile + sr * RS + min(4 * sq + 64 * k, K16)) = st[k];
        __syncthreads();
        const int64_t t1 = t0 + kTileTokens;
        const int n_next = static_cast<int>(min(static_cast<int64_t>(kTileTokens), t_end - t1));
        if (n_next > 0) fetch(t1, n_next);  // in flight during this tile's work

        // scores: this wave's chunks (past Kc: zero rows times a zero query)
        mla_f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
        float4 a[QC];
#pragma unroll
        for (int jj = 0; jj < QC; ++jj)
            a[jj] = *reinterpret_cast<const float4*>(tile + hl * RS + min(16 * (wave + 4 * jj) + 4 * g, K16));
#pragma unroll
        for (int jj = 0; jj < QC; ++jj) {
            s = mfma_f32(a[jj].x, q[jj].x, s);
            s = mfma_f32(a[jj].y, q[jj].y, s);
            s = mfma_f32(a[jj].z, q[jj].z, s);
            s = mfma_f32(a[jj].w, q[jj].w, s);
        }
        red[wave * 64 + lane] = s;
        __syncthreads();
        s = ((red[lane] + red[64 + lane]) + red[128 + lane]) + red[192 + lane];

        // softmax step: lane (head hl, rows 4 g + r); the other lane groups
        // of the head are lanes l ^ 16, l ^ 32, l ^ 48 (permlane swaps)
        float p[4];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = 4 * g + r < n ? s[r] * scale : -INFINITY;
            mt = fmaxf(mt, p[r]);
        }
        mt = cross_groups(mt, [](float x, float y) { return fmaxf(x, y); });
        const float m_new = fmaxf(m_run, mt);
        const float corr = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
        float lt = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = p[r] == -INFINITY ? 0.0f : expf(p[r] - m_new);
            lt += p[r];
        }
        lt = cross_groups(lt, [](float x, float y) { return x + y; });
        l_run = l_run * corr + lt;
        m_run = m_new;

        // values: this wave's column tiles (past nct: the last tile again, never stored)
        const float* vrow = tile + 4 * g * RS + hl;
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const int col = 16 * min(wave + 4 * i, nct - 1);
            acc[i] *= corr;
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i] = mfma_f32(vrow[r * RS + col], p[r], acc[i]);
        }
        n = n_next;
    }
    if (!live) return;
    const int64_t s_idx = blockIdx.x;
    float* dst = part + (s_idx * H + h) * R16;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int ct = wave + 4 * i;
        if (ct < nct)
            *reinterpret_cast<float4*>(dst + 16 * ct + 4 * g) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    }
    if (wave == 0 && g == 0) {
        ml[(s_idx * H + h) * 2] = m_run;
        ml[(s_idx * H + h) * 2 + 1] = l_run;
    }
}

// ------------------------------------------------------------------ merge
// Workgroup (head h, latent columns 256 y ..): latent = sum_s w_s part_s /
// sum_s w_s l_s with w_s = exp(m_s - M) (1 / sum, 0 when the sum is not
// positive, as the reference does).  Each partial is read once; the
// partials are rows of RP (R rounded up to 16) floats.
__global__ __launch_bounds__(kThreads) void mla_merge_kernel(const float* __restrict__ part,
                                                            const float* __restrict__ ml, float* __restrict__ lat,
                                                            int64_t H, int64_t nsplit, int64_t R, int64_t RP) {
    __shared__ float w[kMaxSplits];
    __shared__ float inv_s;
    static_assert(kMaxSplits == 64, "the split weights are one wave's lanes");
    const int64_t h = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (wave == 0) {
        // lane s: split s (a fixed DPP tree for the sum)
        const bool has = lane < nsplit;
        const float m = has ? ml[(static_cast<int64_t>(lane) * H + h) * 2] : -INFINITY;
        const float l = has ? ml[(static_cast<int64_t>(lane) * H + h) * 2 + 1] : 0.0f;
        float M = m;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float ws = m == -INFINITY ? 0.0f : expf(m - M);
        w[lane] = ws;
        const float denom = plm_wave_sum(ws * l);
        if (lane == kSumLane) inv_s = denom > 0.0f ? 1.0f / denom : 0.0f;
    }
    __syncthreads();
    const int64_t c = static_cast<int64_t>(blockIdx.y) * kThreads + tid;
    if (c >= R) return;
    // (loads past the last split read the last one again; their weight is 0)
    const float* src = part + h * RP + c;
    float a = 0.0f;
    for (int64_t s0 = 0; s0 < nsplit; s0 += 16) {
        float vals[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) vals[u] = src[min(s0 + u, nsplit - 1) * H * RP];
#pragma unroll
        for (int u = 0; u < 16; ++u) a = fmaf(w[min(s0 + u, static_cast<int64_t>(kMaxSplits) - 1)], vals[u], a);
    }
    lat[h * R + c] = a * inv_s;
}

// ------------------------------------------------------------------ value rows
// out[h][j] = latent[h] . wkv_b[h][nope + j]: grid (ceil(v / 8), H), two
// rows per wave, every row's loads issued before the sums (VEC: float4 loads,
// R % 4 == 0 and aligned).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void mla_value_kernel(const float* __restrict__ wkv_b,
                                                            const float* __restrict__ lat, float* __restrict__ out,
                                                            int64_t nope, int64_t R, int64_t v) {
    constexpr int kRows = 2;
    const int lane = threadIdx.x & 63;
    const int64_t h = blockIdx.y;
    const int64_t j0 = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6)) * kRows;
    if (j0 >= v) return;
    const float* x = lat + h * R;
    const float* w0 = wkv_b + (h * (nope + v) + nope) * R;
    float acc[kRows] = {};
    if constexpr (VEC) {
        const int64_t R4 = R / 4;
        for (int64_t k = lane; k < R4; k += 64) {
            const float4 xv = reinterpret_cast<const float4*>(x)[k];
            float4 wv[kRows];
#pragma unroll
            for (int i = 0; i < kRows; ++i)
                wv[i] = reinterpret_cast<const float4*>(w0 + min(j0 + i, v - 1) * R)[k];
#pragma unroll
            for (int i = 0; i < kRows; ++i) {
                acc[i] = fmaf(wv[i].x, xv.x, acc[i]);
                acc[i] = fmaf(wv[i].y, xv.y, acc[i]);
                acc[i] = fmaf(wv[i].z, xv.z, acc[i]);
                acc[i] = fmaf(wv[i].w, xv.w, acc[i]);
            }
        }
    } else {
        for (int64_t k = lane; k < R; k += 64) {
            const float xv = x[k];
#pragma unroll
            for (int i = 0; i < kRows; ++i) acc[i] = fmaf(w0[min(j0 + i, v - 1) * R + k], xv, acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        const float t = plm_wave_sum(acc[i]);
        if (lane == kSumLane && j0 + i < v) out[h * v + j0 + i] = t;
    }
}

// ------------------------------------------------------------------ block helpers
// y[n] = W[n] . x, one wave per row; VEC: float4 loads (K % 4 == 0, aligned).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void f32_gemv_kernel(const float* __restrict__ W, const float* __restrict__ x,
                                                           float* __restrict__ y, int64_t N, int64_t K) {
    const int lane = threadIdx.x & 63;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (n >= N) return;
    const float* row = W + n * K;
    float acc = 0.0f;
    if constexpr (VEC) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
        const float4* x4 = reinterpret_cast<const float4*>(x);
        for (int64_t k = lane; k < K / 4; k += 64) {
            const float4 a = r4[k], b = x4[k];
            acc = fmaf(a.x, b.x, acc);
            acc = fmaf(a.y, b.y, acc);
            acc = fmaf(a.z, b.z, acc);
            acc = fmaf(a.w, b.w, acc);
        }
    } else {
        for (int64_t k = lane; k < K; k += 64) acc = fmaf(row[k], x[k], acc);
    }
    acc = plm_wave_sum(acc);
    if (lane == kSumLane) y[n] = acc;
}

// y[n] = W[n] . x for K % 4 == 0 and 16-byte aligned W and x: a workgroup
// owns kGemvRows rows and its waves split K (float4 k on wave (k / 64) % 4),
// so each activation load serves kGemvRows weight loads; kGemvU steps of
// loads are issued before their fmas.  The wave sums are added in wave
// order.
constexpr int kGemvRows = 4;
constexpr int kGemvU = 4;
__global__ __launch_bounds__(kThreads) void f32_gemv_rows_kernel(const float* __restrict__ W,
                                                                const float* __restrict__ x, float* __restrict__ y,
                                                                int64_t N, int64_t K) {
    __shared__ float red[kThreads / 64][kGemvRows];
    const int wave = static_cast<int>(threadIdx.x >> 6);
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kGemvRows;
    const int64_t K4 = K / 4;
    const float4* r4[kGemvRows];
#pragma unroll
    for (int i = 0; i < kGemvRows; ++i)
        r4[i] = reinterpret_cast<const float4*>(W + min(n0 + i, N - 1) * K);  // rows past N re-read the last
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float acc[kGemvRows];
#pragma unroll
    for (int i = 0; i < kGemvRows; ++i) acc[i] = 0.0f;
    for (int64_t k0 = threadIdx.x; k0 < K4; k0 += static_cast<int64_t>(kThreads) * kGemvU) {
        float4 xv[kGemvU], wv[kGemvU][kGemvRows];
#pragma unroll
        for (int u = 0; u < kGemvU; ++u) {
            const int64_t k = min(k0 + static_cast<int64_t>(u) * kThreads, K4 - 1);  // in range; dropped below
            xv[u] = x4[k];
#pragma unroll
            for (int i = 0; i < kGemvRows; ++i) wv[u][i] = r4[i][k];
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the steps before the first fma
#pragma unroll
        for (int u = 0; u < kGemvU; ++u) {
            if (k0 + static_cast<int64_t>(u) * kThreads >= K4) xv[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int i = 0; i < kGemvRows; ++i) {
                if (k0 + static_cast<int64_t>(u) * kThreads >= K4) wv[u][i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                acc[i] = fmaf(wv[u][i].x, xv[u].x, acc[i]);
                acc[i] = fmaf(wv[u][i].y, xv[u].y, acc[i]);
                acc[i] = fmaf(wv[u][i].z, xv[u].z, acc[i]);
                acc[i] = fmaf(wv[u][i].w, xv[u].w, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kGemvRows; ++i) {
        const float t = plm_wave_sum(acc[i]);
        if (lane == kSumLane) red[wave][i] = t;
    }
    __syncthreads();
    if (threadIdx.x < kGemvRows && n0 + threadIdx.x < N) {
        const int i = static_cast<int>(threadIdx.x);
        y[n0 + i] = ((red[0][i] + red[1][i]) + red[2][i]) + red[3][i];
    }
}

// v = v * (1 / sqrt(mean(v^2) + eps)) * w (ds_forward.cpp:610-619), one workgroup.
__device__ void rms_norm_block(const float* v, const float* w, float* out, int64_t dim, float eps) {
    __shared__ float red[kThreads / 64];
    const int tid = threadIdx.x;
    float ss = 0.0f;
    for (int64_t i = tid; i < dim; i += kThreads) ss = fmaf(v[i], v[i], ss);
    ss = plm_wave_sum(ss);
    if ((tid & 63) == kSumLane) red[tid >> 6] = ss;
    __syncthreads();
    const float total = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = 1.0f / sqrtf(total / static_cast<float>(dim) + eps);
    for (int64_t i = tid; i < dim; i += kThreads) out[i] = v[i] * inv * w[i];
    __syncthreads();
}


// q [H][nope + rope] -> q_nope [H][nope], q_pe [H][rope] with RoPE.
__global__ __launch_bounds__(kThreads) void mla_q_split_kernel(const float* __restrict__ q, float* __restrict__ q_nope,
                                                              float* __restrict__ q_pe, const float* __restrict__ cs,
                                                              const float* __restrict__ sn, int64_t H, int64_t nope,
                                                              int64_t rope) {
    const int64_t w = nope + rope;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < H * nope) {
        const int64_t h = i / nope, d = i - h * nope;
        q_nope[i] = q[h * w + d];
    }
    const int64_t pairs = rope / 2;
    if ((rope & 1) == 0 && i < H * pairs) {
        const int64_t h = i / pairs, p = i - h * pairs;
        rope_pair(q + h * w + nope, q_pe + h * rope, p, cs, sn);
    }
    if ((rope & 1) != 0 && i < H * rope) {  // an odd rope width is left unrotated (ds_forward.cpp:628-630)
        const int64_t h = i / rope, d = i - h * rope;
        q_pe[i] = q[h * w + nope + d];
    }
}

// The two norms after the q_a / kv_a projections, one workgroup each:
// q_low in place (workgroup 0), and the new cache row (workgroup 1).
__global__ __launch_bounds__(kThreads) void mla_norms_kernel(float* __restrict__ q_low,
                                                            const float* __restrict__ q_norm, int64_t q_rank,
                                                            const float* __restrict__ kvraw,
                                                            const float* __restrict__ kv_norm, float* __restrict__ kv_row,
                                                            float* __restrict__ pe_row, const float* __restrict__ cs,
                                                            const float* __restrict__ sn, int64_t R, int64_t rope,
                                                            float eps) {
    if (blockIdx.x == 0) {
        rms_norm_block(q_low, q_norm, q_low, q_rank, eps);
        return;
    }
    rms_norm_block(kvraw, kv_norm, kv_row, R, eps);
    if ((rope & 1) == 0) {
        for (int64_t p = threadIdx.x; p < rope / 2; p += kThreads) rope_pair(kvraw + R, pe_row, p, cs, sn);
    } else {
        for (int64_t d = threadIdx.x; d < rope; d += kThreads) pe_row[d] = kvraw[R + d];
    }
}

int gemv(const float* W, const float* x, float* y, int64_t N, int64_t K, hipStream_t st) {
    static_assert(kThreads == 256, "four waves add their sums in f32_gemv_rows_kernel");
    const bool vec = K % 4 == 0 && plm::aligned16(W) && plm::aligned16(x);
    if (vec && K / 4 >= static_cast<int64_t>(kThreads) * kGemvU) {
        // rows of at least 4096 values: the row groups (q_b 24576x1536 was
        // 1.7 us faster one wave per row)
        hipLaunchKernelGGL(f32_gemv_rows_kernel, dim3(static_cast<unsigned>(plm::ceil_div(N, kGemvRows))),
                           dim3(kThreads), 0, st, W, x, y, N, K);
    } else if (vec) {
        hipLaunchKernelGGL(f32_gemv_kernel<true>, dim3(static_cast<unsigned>(plm::ceil_div(N, kThreads / 64))),
                           dim3(kThreads), 0, st, W, x, y, N, K);
    } else {
        hipLaunchKernelGGL(f32_gemv_kernel<false>, dim3(static_cast<unsigned>(plm::ceil_div(N, kThreads / 64))),
                           dim3(kThreads), 0, st, W, x, y, N, K);
    }
    return plm::check_launch("f32 gemv");
}

// Tokens per split: a multiple of 16, at least two tiles (the next tile's
// loads overlap the current one's work), at most kMaxSplits splits.
int64_t tokens_per_split(int64_t L) {
    return std::max<int64_t>(2 * kTileTokens,
                             plm::ceil_div(plm::ceil_div(L, kMaxSplits), kTileTokens) * kTileTokens);
}

// The flash workspace, in floats, every array 16-byte aligned: q_abs [H][R],
// the partials [nsplit][H][R16], (max, sum) [nsplit][H][2], latent [H][R].
struct FlashLayout {
    int64_t per, nsplit, part, ml, lat, total;
};

FlashLayout flash_layout(int64_t H, int64_t L, int64_t R) {
    auto align4 = [](int64_t n) { return (n + 3) & ~int64_t(3); };
    FlashLayout f;
    f.per = tokens_per_split(L);
    f.nsplit = plm::ceil_div(L, f.per);
    f.part = align4(H * R);
    f.ml = f.part + f.nsplit * H * split_shape(R, 0).R16;
    f.lat = align4(f.ml + f.nsplit * H * 2);
    f.total = f.lat + H * R;
    return f;
}

size_t flash_workspace_bytes(int64_t H, int64_t L, int64_t R) {
    return static_cast<size_t>(flash_layout(H, L, R).total) * sizeof(float);
}

// The split kernel's instances: <QC, NT> with QC >= ceil(K16 / 64) and
// NT >= ceil(R16 / 64).
template <int QC, int NT>
int launch_split(dim3 grid, size_t lds, hipStream_t st, bool vec, const float* q_abs, const float* q_pe, const float* kv,
                 const float* pe, float* part, float* ml, int64_t H, int64_t L, int64_t R, int64_t rope, float scale,
                 int64_t per) {
    if (lds > 64 * 1024) {
        static bool raised[2] = {false, false};  // per instance and VEC
        if (!raised[vec]) {
            const void* fn = vec ? reinterpret_cast<const void*>(&mla_split_kernel<QC, NT, true>)
                                 : reinterpret_cast<const void*>(&mla_split_kernel<QC, NT, false>);
            if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
                return plm::fail(-1, "mla split kernel: LDS attribute refused");
            raised[vec] = true;
        }
    }
    if (vec)
        hipLaunchKernelGGL((mla_split_kernel<QC, NT, true>), grid, dim3(kThreads), lds, st, q_abs, q_pe, kv, pe, part,
                           ml, H, L, R, rope, scale, per);
    else
        hipLaunchKernelGGL((mla_split_kernel<QC, NT, false>), grid, dim3(kThreads), lds, st, q_abs, q_pe, kv, pe, part,
                           ml, H, L, R, rope, scale, per);
    return plm::check_launch("mla split kernel");
}

// The MLA launches; ws holds flash_workspace_bytes.
// The absorbed-query kernel's 4-wide instance (the one that can also write
// the RoPE'd q_pe).
bool qabs4_ok(int64_t R, const float* wkv_b) { return R % 4 == 0 && plm::aligned16(wkv_b); }

// With rope_in set, q_nope rows are q_stride floats apart and the q_abs
// kernel writes q_pe (q_pe_out, which q_pe must name) from rope_in; only
// when qabs4_ok.
int flash(const float* q_nope, const float* q_pe, const float* kv, const float* pe, const float* wkv_b, float* out,
          int64_t H, int64_t L, int64_t nope, int64_t rope, int64_t R, int64_t v, float scale, float* ws,
          hipStream_t st, int64_t q_stride = 0, const float* rope_in = nullptr, float* q_pe_out = nullptr,
          const float* cs = nullptr, const float* sn = nullptr) {
    if (rope_in != nullptr && (!qabs4_ok(R, wkv_b) || q_pe_out != q_pe)) return plm::fail(-2, "fused q split");
    const FlashLayout f = flash_layout(H, L, R);
    const int64_t per = f.per, nsplit = f.nsplit;
    const SplitShape sh = split_shape(R, rope);
    float* q_abs = ws;
    float* part = ws + f.part;
    float* ml = ws + f.ml;
    float* lat = ws + f.lat;
    if (qabs4_ok(R, wkv_b))
        hipLaunchKernelGGL(mla_qabs4_kernel<kQabsWaves>,
                           dim3(static_cast<unsigned>(H), static_cast<unsigned>(plm::ceil_div(R, 256))),
                           dim3(kQabsWaves * 64), 0, st, q_nope, q_stride > 0 ? q_stride : nope, wkv_b, q_abs, nope,
                           R, v, rope_in, q_pe_out, cs, sn, rope);
    else
        hipLaunchKernelGGL(mla_qabs_kernel, dim3(static_cast<unsigned>(H), static_cast<unsigned>(plm::ceil_div(R, 64))),
                           dim3(kThreads), 0, st, q_nope, wkv_b, q_abs, nope, R, v);
    int code = plm::check_launch("mla q_abs kernel");
    if (code != 0) return code;
    const dim3 sgrid(static_cast<unsigned>(nsplit), static_cast<unsigned>(plm::ceil_div(H, kHeadsPerGroup)));
    // q_pe / pe are not read when rope is 0 (the reference still requires them)
    const bool vec = R % 4 == 0 && rope % 4 == 0 && plm::aligned16(q_abs) && plm::aligned16(kv) &&
                     (rope == 0 || (plm::aligned16(q_pe) && plm::aligned16(pe)));
    const int64_t qc = plm::ceil_div(sh.K16, 64), nt = plm::ceil_div(sh.R16, 64);
    const size_t lds = split_lds_bytes(R, rope);
    if (qc <= 3 && nt <= 2)
        code = launch_split<3, 2>(sgrid, lds, st, vec, q_abs, q_pe, kv, pe, part, ml, H, L, R, rope, scale, per);
    else if (qc <= 9 && nt <= 8)
        code = launch_split<9, 8>(sgrid, lds, st, vec, q_abs, q_pe, kv, pe, part, ml, H, L, R, rope, scale, per);
    else
        code = launch_split<20, 16>(sgrid, lds, st, vec, q_abs, q_pe, kv, pe, part, ml, H, L, R, rope, scale, per);
    if (code != 0) return code;
    hipLaunchKernelGGL(mla_merge_kernel, dim3(static_cast<unsigned>(H), static_cast<unsigned>(plm::ceil_div(R, kThreads))),
                       dim3(kThreads), 0, st, part, ml, lat, H, nsplit, R, sh.R16);
    if ((code = plm::check_launch("mla merge kernel")) != 0) return code;
    const dim3 vgrid(static_cast<unsigned>(plm::ceil_div(v, 8)), static_cast<unsigned>(H));
    if (R % 4 == 0 && plm::aligned16(wkv_b) && plm::aligned16(lat))
        hipLaunchKernelGGL(mla_value_kernel<true>, vgrid, dim3(kThreads), 0, st, wkv_b, lat, out, nope, R, v);
    else
        hipLaunchKernelGGL(mla_value_kernel<false>, vgrid, dim3(kThreads), 0, st, wkv_b, lat, out, nope, R, v);
    return plm::check_launch("mla value kernel");
}

bool device_limits_ok(int64_t R, int64_t rope) { return R <= kMaxRank && rope <= kMaxRope; }

}  // namespace

// ====================================================================== C ABI

PLM_EXPORT int ds_mla_attention_flash_forward(const float* q_nope, const float* q_pe, const float* kv_cache,
                                              const float* pe_cache, const float* wkv_b, float* output_heads,
                                              int64_t num_heads, int64_t cache_len, int64_t qk_nope_dim,
                                              int64_t qk_rope_dim, int64_t kv_lora_rank, int64_t v_head_dim,
                                              float softmax_scale) {
    if (!q_nope || !q_pe || !kv_cache || !pe_cache || !wkv_b || !output_heads) return plm::fail(1, "null pointer");
    if (num_heads <= 0 || cache_len <= 0 || qk_nope_dim < 0 || qk_rope_dim < 0 || kv_lora_rank <= 0 || v_head_dim <= 0)
        return plm::fail(2, "bad dimensions");
    if (!device_limits_ok(kv_lora_rank, qk_rope_dim))
        return plm::fail(2, "kv_lora_rank %lld / qk_rope_dim %lld beyond the device kernel's %lld / %lld",
                         static_cast<long long>(kv_lora_rank), static_cast<long long>(qk_rope_dim),
                         static_cast<long long>(kMaxRank), static_cast<long long>(kMaxRope));
    float* ws = static_cast<float*>(plm::workspace(flash_workspace_bytes(num_heads, cache_len, kv_lora_rank)));
    if (ws == nullptr) return -3;
    return flash(q_nope, q_pe, kv_cache, pe_cache, wkv_b, output_heads, num_heads, cache_len, qk_nope_dim,
                 qk_rope_dim, kv_lora_rank, v_head_dim, softmax_scale, ws, plm::current_stream());
}

namespace {

// The attention block after its projections are chosen (ds_forward.cpp:647-782):
// project_a fills q_low [q_rank] and kvraw [R + rope] from the hidden state,
// project_qb fills q [H (nope + rope)] from the normalised q_low, project_o
// fills the output from heads [H v].  ws: block_workspace_floats floats.
struct BlockDims {
    int64_t hidden, q_rank, R, H, nope, rope, v, prev;
};

int64_t block_scratch_floats(const BlockDims& d) {
    const int64_t scratch = d.q_rank + d.H * (d.nope + d.rope) + d.H * d.nope + d.H * d.rope + (d.R + d.rope) + d.H * d.v;
    return (scratch + 63) & ~int64_t(63);
}

size_t block_workspace_bytes(const BlockDims& d) {
    return static_cast<size_t>(block_scratch_floats(d)) * sizeof(float) + flash_workspace_bytes(d.H, d.prev + 1, d.R);
}

template <class ProjectA, class ProjectQb, class ProjectO>
int attention_block(const BlockDims& d, ProjectA&& project_a, ProjectQb&& project_qb, ProjectO&& project_o,
                    const float* kv_b_weight, const float* q_norm_weight, const float* kv_norm_weight,
                    const float* previous_kv_cache, const float* previous_pe_cache, const float* rope_cos,
                    const float* rope_sin, float* next_kv_cache, float* next_pe_cache, float rms_eps,
                    float softmax_scale, float* ws, hipStream_t st) {
    const int64_t H = d.H, nope = d.nope, rope = d.rope, R = d.R, v = d.v, qw = nope + rope, L = d.prev + 1;
    float* q_low = ws;
    float* q = q_low + d.q_rank;
    float* qn = q + H * qw;
    float* qp = qn + H * nope;
    float* kvraw = qp + H * rope;
    float* heads = kvraw + R + rope;
    float* fws = ws + block_scratch_floats(d);

    int code = project_a(q_low, kvraw);
    if (code != 0) return code;
    // the new row (RMSNorm of the latent, RoPE of the pe part) goes after
    // the previous rows, which are copied below into other buffers only
    hipLaunchKernelGGL(mla_norms_kernel, dim3(2), dim3(kThreads), 0, st, q_low, q_norm_weight, d.q_rank, kvraw,
                       kv_norm_weight, next_kv_cache + d.prev * R, next_pe_cache + d.prev * rope, rope_cos, rope_sin, R,
                       rope, rms_eps);
    if ((code = plm::check_launch("mla norms")) != 0) return code;
    if ((code = project_qb(q_low, q)) != 0) return code;
    // q_nope and the RoPE'd q_pe: read and written by the q_abs kernel when
    // its 4-wide instance runs, else split out here
    const bool fused_q = qabs4_ok(R, kv_b_weight);
    if (!fused_q) {
        const int64_t qn_threads = std::max(H * nope, H * rope);
        hipLaunchKernelGGL(mla_q_split_kernel,
                           dim3(static_cast<unsigned>(plm::ceil_div(std::max<int64_t>(qn_threads, 1), kThreads))),
                           dim3(kThreads), 0, st, q, qn, qp, rope_cos, rope_sin, H, nope, rope);
        if ((code = plm::check_launch("mla q split")) != 0) return code;
    }
    // the previous rows, then the new one (ds_forward.cpp:716-744)
    if (d.prev > 0) {
        hipError_t err = hipSuccess;
        if (next_kv_cache != previous_kv_cache)
            err = hipMemcpyAsync(next_kv_cache, previous_kv_cache,
                                 static_cast<size_t>(d.prev * R) * sizeof(float), hipMemcpyDeviceToDevice, st);
        if (err == hipSuccess && rope > 0 && next_pe_cache != previous_pe_cache)
            err = hipMemcpyAsync(next_pe_cache, previous_pe_cache,
                                 static_cast<size_t>(d.prev * rope) * sizeof(float), hipMemcpyDeviceToDevice, st);
        if (err != hipSuccess) return plm::hip_fail(err, "previous cache copy");
    }
    code = fused_q ? flash(q, qp, next_kv_cache, next_pe_cache, kv_b_weight, heads, H, L, nope, rope, R, v,
                           softmax_scale, fws, st, qw, q + nope, qp, rope_cos, rope_sin)
                   : flash(qn, qp, next_kv_cache, next_pe_cache, kv_b_weight, heads, H, L, nope, rope, R, v,
                           softmax_scale, fws, st);
    if (code != 0) return code > 0 ? 100 + code : code;
    return project_o(heads);
}

}  // namespace

PLM_EXPORT int ds_attention_block_forward_f32(
    void* handle, const float* hidden_in, const float* q_a_weight, const float* q_b_weight, const float* kv_a_weight,
    const float* kv_b_weight, const float* o_weight, const float* q_norm_weight, const float* kv_norm_weight,
    const float* previous_kv_cache, const float* previous_pe_cache, const float* rope_cos, const float* rope_sin,
    float* next_kv_cache, float* next_pe_cache, float* hidden_out, int64_t hidden_dim, int64_t q_lora_rank,
    int64_t kv_lora_rank, int64_t num_heads, int64_t qk_nope_dim, int64_t qk_rope_dim, int64_t v_head_dim,
    int64_t previous_len, float rms_eps, float softmax_scale) {
    if (!handle || !hidden_in || !q_a_weight || !q_b_weight || !kv_a_weight || !kv_b_weight || !o_weight ||
        !q_norm_weight || !kv_norm_weight || !rope_cos || !rope_sin || !next_kv_cache || !next_pe_cache || !hidden_out)
        return plm::fail(1, "null pointer");
    if (hidden_dim <= 0 || q_lora_rank <= 0 || kv_lora_rank <= 0 || num_heads <= 0 || qk_nope_dim < 0 ||
        qk_rope_dim < 0 || v_head_dim <= 0 || previous_len < 0)
        return plm::fail(2, "bad dimensions");
    if (previous_len > 0 && (!previous_kv_cache || !previous_pe_cache))
        return plm::fail(3, "previous caches are null with previous_len %lld", static_cast<long long>(previous_len));
    if (!device_limits_ok(kv_lora_rank, qk_rope_dim)) return 102;  // the flash call's dimension code, offset by 100
    const BlockDims d{hidden_dim, q_lora_rank, kv_lora_rank, num_heads, qk_nope_dim, qk_rope_dim, v_head_dim,
                      previous_len};
    hipStream_t st = plm::current_stream();
    float* ws = static_cast<float*>(plm::workspace(block_workspace_bytes(d)));
    if (ws == nullptr) return -3;
    const int64_t qw = qk_nope_dim + qk_rope_dim;
    auto project_a = [&](float* q_low, float* kvraw) {
        const int code = gemv(q_a_weight, hidden_in, q_low, q_lora_rank, hidden_dim, st);
        return code != 0 ? code : gemv(kv_a_weight, hidden_in, kvraw, kv_lora_rank + qk_rope_dim, hidden_dim, st);
    };
    auto project_qb = [&](const float* q_low, float* q) {
        return gemv(q_b_weight, q_low, q, num_heads * qw, q_lora_rank, st);
    };
    auto project_o = [&](const float* heads) {
        return gemv(o_weight, heads, hidden_out, hidden_dim, num_heads * v_head_dim, st);
    };
    const int code = attention_block(d, project_a, project_qb, project_o, kv_b_weight, q_norm_weight, kv_norm_weight,
                                     previous_kv_cache, previous_pe_cache, rope_cos, rope_sin, next_kv_cache,
                                     next_pe_cache, rms_eps, softmax_scale, ws, st);
    if (code != 0) return code;
    return plm_ds_session_note_fused_attention(handle);
}

// The FP8 attention of one decode token (fp8_source.py:6337-6454 at one
// token): q_a and kv_a in one FP8 launch on the bf16 hidden state, q_b and o
// as FP8 linears on fp32 activations (the reference's native FP8 linear takes
// fp32), kv_b dequantized to fp32 beforehand as the reference loads it.
PLM_EXPORT int ds_fp8_attention_block_bf16x_f32(
    const uint16_t* hidden_bf16, const uint8_t* q_a_weight, const float* q_a_scale_inv, const uint8_t* q_b_weight,
    const float* q_b_scale_inv, const uint8_t* kv_a_weight, const float* kv_a_scale_inv, const float* kv_b_weight,
    const uint8_t* o_weight, const float* o_scale_inv, const float* q_norm_weight, const float* kv_norm_weight,
    const float* previous_kv_cache, const float* previous_pe_cache, const float* rope_cos, const float* rope_sin,
    float* next_kv_cache, float* next_pe_cache, float* hidden_out, int64_t hidden_dim, int64_t q_lora_rank,
    int64_t kv_lora_rank, int64_t num_heads, int64_t qk_nope_dim, int64_t qk_rope_dim, int64_t v_head_dim,
    int64_t previous_len, float rms_eps, float softmax_scale) {
    if (!hidden_bf16 || !q_a_weight || !q_a_scale_inv || !q_b_weight || !q_b_scale_inv || !kv_a_weight ||
        !kv_a_scale_inv || !kv_b_weight || !o_weight || !o_scale_inv || !q_norm_weight || !kv_norm_weight ||
        !rope_cos || !rope_sin || !next_kv_cache || !next_pe_cache || !hidden_out)
        return plm::fail(1, "null pointer");
    if (hidden_dim <= 0 || q_lora_rank <= 0 || kv_lora_rank <= 0 || num_heads <= 0 || qk_nope_dim < 0 ||
        qk_rope_dim < 0 || v_head_dim <= 0 || previous_len < 0)
        return plm::fail(2, "bad dimensions");
    if (previous_len > 0 && (!previous_kv_cache || !previous_pe_cache))
        return plm::fail(3, "previous caches are null with previous_len %lld", static_cast<long long>(previous_len));
    if (!device_limits_ok(kv_lora_rank, qk_rope_dim)) return 102;
    const BlockDims d{hidden_dim, q_lora_rank, kv_lora_rank, num_heads, qk_nope_dim, qk_rope_dim, v_head_dim,
                      previous_len};
    hipStream_t st = plm::current_stream();
    float* ws = static_cast<float*>(plm::workspace(block_workspace_bytes(d)));
    if (ws == nullptr) return -3;
    const int64_t qw = qk_nope_dim + qk_rope_dim;
    auto cols = [](int64_t k) { return plm::ceil_div(k, 128); };
    auto project_a = [&](float* q_low, float* kvraw) {
        const uint64_t w[2] = {reinterpret_cast<uint64_t>(q_a_weight), reinterpret_cast<uint64_t>(kv_a_weight)};
        const uint64_t s[2] = {reinterpret_cast<uint64_t>(q_a_scale_inv), reinterpret_cast<uint64_t>(kv_a_scale_inv)};
        const uint64_t o[2] = {reinterpret_cast<uint64_t>(q_low), reinterpret_cast<uint64_t>(kvraw)};
        const int64_t rows[2] = {q_lora_rank, kv_lora_rank + qk_rope_dim};
        return fp8_e4m3_block_linear_many_bf16x_f32(w, s, hidden_bf16, o, rows, 2, 1, hidden_dim, cols(hidden_dim));
    };
    auto project_qb = [&](const float* q_low, float* q) {
        return fp8_e4m3_block_linear_f32(q_b_weight, q_b_scale_inv, q_low, q, 1, num_heads * qw, q_lora_rank,
                                         cols(q_lora_rank));
    };
    auto project_o = [&](const float* heads) {
        return fp8_e4m3_block_linear_f32(o_weight, o_scale_inv, heads, hidden_out, 1, hidden_dim,
                                         num_heads * v_head_dim, cols(num_heads * v_head_dim));
    };
    return attention_block(d, project_a, project_qb, project_o, kv_b_weight, q_norm_weight, kv_norm_weight,
                           previous_kv_cache, previous_pe_cache, rope_cos, rope_sin, next_kv_cache, next_pe_cache,
                           rms_eps, softmax_scale, ws, st);
}
