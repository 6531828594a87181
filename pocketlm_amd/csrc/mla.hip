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
//   mla_split_kernel      flash-decode partials: workgroup (split, 16 heads)
//                         walks its tokens in tiles of 16 rows staged in LDS
//                         (each latent row is read once for 16 heads); a
//                         thread owns one head's 1/16 of the latent columns,
//                         with a running max / sum per head.
//   mla_merge_out_kernel  rescales the splits to the global max, divides by
//                         the sum (1 / sum, 0 when the sum is not positive, as
//                         the reference does), and applies the value rows of
//                         kv_b to the latent: workgroup (head, 32 outputs).
//
// The block: fp32 GEMVs (one wave per row, float4 loads, a fixed DPP sum),
// RMSNorm and RoPE kernels, the new cache row appended after the previous
// rows, then the three MLA kernels and the output projection; every launch
// on the caller's stream.
#include <cmath>
#include <algorithm>
#include <cstring>

#include "common.h"

int plm_ds_session_note_fused_attention(void* handle);

namespace {

constexpr int kThreads = 256;
constexpr int kHeadsPerGroup = 16;  // heads of one split workgroup
constexpr int kTileTokens = 16;     // latent rows staged per step
constexpr int64_t kMaxRank = 1024;  // 16 chunks of at most 64 columns
constexpr int64_t kMaxRope = 256;   // 16 chunks of at most 16
constexpr int kMaxSplits = 64;

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

// ------------------------------------------------------------------ split
// Thread (head tid / 16 of the group, column chunk tid % 16): it holds the
// CPT query values of its chunk in registers (and PPT of the rope part), dots
// them with each staged row's chunk, and the 16 chunks' partial dots are
// added across the head's 16 lanes (xor shuffles), so every lane of a head
// sees all 16 scores of the tile.  The same thread then accumulates its
// chunk of the head's latent with those weights.  LDS holds the tile's rows
// chunk by chunk, each chunk padded by one float (no bank conflicts between
// the 16 chunks).
constexpr int kChunks = 16;

__host__ __device__ constexpr int64_t split_lds_floats(int cpt, int ppt) {
    return static_cast<int64_t>(kTileTokens) * kChunks * ((cpt + 4) + (ppt + 4)) + kHeadsPerGroup * kTileTokens;
}

size_t split_lds_bytes(int cpt, int ppt) { return static_cast<size_t>(split_lds_floats(cpt, ppt)) * sizeof(float); }

template <int CPT, int PPT>
__global__ __launch_bounds__(kThreads) void mla_split_kernel(const float* __restrict__ q_abs,
                                                            const float* __restrict__ q_pe,
                                                            const float* __restrict__ kv, const float* __restrict__ pe,
                                                            float* __restrict__ part, float* __restrict__ ml,
                                                            int64_t H, int64_t L, int64_t R, int64_t rope, float scale,
                                                            int64_t per_split) {
    extern __shared__ float4 sm4[];
    float* sm = reinterpret_cast<float*>(sm4);
    constexpr int CS = CPT + 4, PS = PPT + 4;  // 16-byte aligned chunks, staggered over the banks
    static_assert(CPT % 4 == 0 && PPT % 4 == 0, "chunks of whole float4s");
    float* kv_t = sm;                                // [16 rows][16 chunks][CS]
    float* pe_t = kv_t + kTileTokens * kChunks * CS;  // [16 rows][16 chunks][PS]
    float* pw = pe_t + kTileTokens * kChunks * PS;    // [16 heads][16 rows]: scores, then weights
    const int tid = threadIdx.x;
    const int hh = tid >> 4, cq = tid & 15;
    const int64_t h = static_cast<int64_t>(blockIdx.y) * kHeadsPerGroup + hh;
    const bool live = h < H;
    const int64_t t_begin = static_cast<int64_t>(blockIdx.x) * per_split;
    const int64_t t_end = min(L, t_begin + per_split);
    const bool vec4 = CPT % 4 == 0 && (R & 3) == 0 && (reinterpret_cast<uintptr_t>(kv) & 15) == 0;
    float q[CPT], qr[PPT], acc[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int64_t c = static_cast<int64_t>(cq) * CPT + i;
        q[i] = live && c < R ? q_abs[h * R + c] : 0.0f;
        acc[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
        const int64_t c = static_cast<int64_t>(cq) * PPT + i;
        qr[i] = live && c < rope ? q_pe[h * rope + c] : 0.0f;
    }
    float m_run = -INFINITY, l_run = 0.0f;

    for (int64_t t0 = t_begin; t0 < t_end; t0 += kTileTokens) {
        const int n = static_cast<int>(min(static_cast<int64_t>(kTileTokens), t_end - t0));
        // thread (row tid / 16, chunk tid % 16) stages that chunk of the row:
        // every load is issued before the first store
        {
            const int sr = tid >> 4, sc0 = tid & 15;
            const bool row_in = sr < n;
            const int64_t row = t0 + (row_in ? sr : 0);
            const float* src = kv + row * R + static_cast<int64_t>(sc0) * CPT;
            const int64_t left = R - static_cast<int64_t>(sc0) * CPT;  // columns of this chunk inside R
            float vals[CPT];
            if (vec4 && left >= CPT) {
#pragma unroll
                for (int i = 0; i < CPT / 4; ++i) {
                    const float4 f = reinterpret_cast<const float4*>(src)[i];
                    vals[4 * i] = f.x;
                    vals[4 * i + 1] = f.y;
                    vals[4 * i + 2] = f.z;
                    vals[4 * i + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < CPT; ++i) vals[i] = i < left ? src[i] : 0.0f;
            }
            float pvals[PPT];
            const float* psrc = pe + row * rope + static_cast<int64_t>(sc0) * PPT;
            const int64_t pleft = rope - static_cast<int64_t>(sc0) * PPT;
#pragma unroll
            for (int i = 0; i < PPT; ++i) pvals[i] = i < pleft ? psrc[i] : 0.0f;
            __syncthreads();  // the previous tile's readers are done
            float4* dst = reinterpret_cast<float4*>(kv_t + (sr * kChunks + sc0) * CS);
#pragma unroll
            for (int i = 0; i < CPT / 4; ++i)
                dst[i] = row_in ? make_float4(vals[4 * i], vals[4 * i + 1], vals[4 * i + 2], vals[4 * i + 3])
                                : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            float4* pdst = reinterpret_cast<float4*>(pe_t + (sr * kChunks + sc0) * PS);
#pragma unroll
            for (int i = 0; i < PPT / 4; ++i)
                pdst[i] = row_in ? make_float4(pvals[4 * i], pvals[4 * i + 1], pvals[4 * i + 2], pvals[4 * i + 3])
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        __syncthreads();
        // scores, one token at a time: the chunk's partial dot (latent, then
        // rope part), added over the head's 16 lanes; lane 0 of the head
        // keeps it in pw
        for (int t = 0; t < n; ++t) {
            const float4* k = reinterpret_cast<const float4*>(kv_t + (t * kChunks + cq) * CS);
            const float4* kr = reinterpret_cast<const float4*>(pe_t + (t * kChunks + cq) * PS);
            float d = 0.0f, dr = 0.0f;
#pragma unroll
            for (int i = 0; i < CPT / 4; ++i) {
                const float4 kk = k[i];
                d = fmaf(q[4 * i], kk.x, d);
                d = fmaf(q[4 * i + 1], kk.y, d);
                d = fmaf(q[4 * i + 2], kk.z, d);
                d = fmaf(q[4 * i + 3], kk.w, d);
            }
#pragma unroll
            for (int i = 0; i < PPT / 4; ++i) {
                const float4 kk = kr[i];
                dr = fmaf(qr[4 * i], kk.x, dr);
                dr = fmaf(qr[4 * i + 1], kk.y, dr);
                dr = fmaf(qr[4 * i + 2], kk.z, dr);
                dr = fmaf(qr[4 * i + 3], kk.w, dr);
            }
            float sc = d + dr;
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) sc += __shfl_xor(sc, off);
            if (cq == 0) pw[hh * kTileTokens + t] = sc * scale;
        }
        __syncthreads();
        // softmax step, lane cq of a head taking token cq
        const float st = cq < n ? pw[hh * kTileTokens + cq] : -INFINITY;
        float mt = st;
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off));
        const float m_new = fmaxf(m_run, mt);
        const float corr = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
        const float pt = st == -INFINITY ? 0.0f : expf(st - m_new);
        float lt = pt;
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) lt += __shfl_xor(lt, off);
        l_run = l_run * corr + lt;
        m_run = m_new;
        __syncthreads();  // every score read before the weights replace them
        pw[hh * kTileTokens + cq] = pt;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < CPT; ++i) acc[i] *= corr;
        for (int t = 0; t < n; ++t) {
            const float w = pw[hh * kTileTokens + t];
            const float4* k = reinterpret_cast<const float4*>(kv_t + (t * kChunks + cq) * CS);
#pragma unroll
            for (int i = 0; i < CPT / 4; ++i) {
                const float4 kk = k[i];
                acc[4 * i] = fmaf(w, kk.x, acc[4 * i]);
                acc[4 * i + 1] = fmaf(w, kk.y, acc[4 * i + 1]);
                acc[4 * i + 2] = fmaf(w, kk.z, acc[4 * i + 2]);
                acc[4 * i + 3] = fmaf(w, kk.w, acc[4 * i + 3]);
            }
        }
    }
    if (!live) return;
    const int64_t s_idx = blockIdx.x;
    float* dst = part + (s_idx * H + h) * R;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int64_t c = static_cast<int64_t>(cq) * CPT + i;
        if (c < R) dst[c] = acc[i];
    }
    if (cq == 0) {
        ml[(s_idx * H + h) * 2] = m_run;
        ml[(s_idx * H + h) * 2 + 1] = l_run;
    }
}

// ------------------------------------------------------------------ merge + value rows
// Workgroup (head h, outputs 32 j0 .. 32 j0 + 31): latent = sum_s w_s part_s /
// sum_s w_s l_s with w_s = exp(m_s - M), then out[h][j] = latent . wkv_b[h][nope + j].
__global__ __launch_bounds__(kThreads) void mla_merge_out_kernel(const float* __restrict__ part,
                                                                const float* __restrict__ ml,
                                                                const float* __restrict__ wkv_b,
                                                                float* __restrict__ out, int64_t H, int64_t nsplit,
                                                                int64_t nope, int64_t R, int64_t v) {
    extern __shared__ float lat[];  // [R]
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
    const float inv = inv_s;
    // (loads past the last split read the last one again; their weight is 0)
    for (int64_t c = tid; c < R; c += kThreads) {
        const float* src = part + h * R + c;
        float a = 0.0f;
        for (int64_t s0 = 0; s0 < nsplit; s0 += 16) {
            float vals[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) vals[u] = src[min(s0 + u, nsplit - 1) * H * R];
#pragma unroll
            for (int u = 0; u < 16; ++u) a = fmaf(w[min(s0 + u, static_cast<int64_t>(kMaxSplits) - 1)], vals[u], a);
        }
        lat[c] = a * inv;
    }
    __syncthreads();
    const float* wv = wkv_b + (h * (nope + v) + nope) * R;
    const int64_t j_end = min(v, static_cast<int64_t>(blockIdx.y) * 32 + 32);
    for (int64_t j = static_cast<int64_t>(blockIdx.y) * 32 + wave; j < j_end; j += 4) {
        const float* row = wv + j * R;
        float a = 0.0f;
        for (int64_t c0 = lane; c0 < R; c0 += 64 * 8) {
            float vals[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) vals[u] = row[min(c0 + 64 * u, R - 1)];
#pragma unroll
            for (int u = 0; u < 8; ++u) a = fmaf(c0 + 64 * u < R ? lat[c0 + 64 * u] : 0.0f, vals[u], a);
        }
        a = plm_wave_sum(a);
        if (lane == kSumLane) out[h * v + j] = a;
    }
}

// ------------------------------------------------------------------ block helpers
// y[n] = W[n] . x: one wave per row; VEC: float4 loads (K % 4 == 0, aligned).
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

// RoPE on pairs (x0, x1) of each group of `dim` values (ds_forward.cpp:621-645).
__device__ __forceinline__ void rope_pair(const float* in, float* out, int64_t pair, const float* cs, const float* sn) {
    const float x0 = in[2 * pair], x1 = in[2 * pair + 1];
    const float c = cs[pair], s = sn[pair];
    out[2 * pair] = x0 * c - x1 * s;
    out[2 * pair + 1] = x0 * s + x1 * c;
}

__global__ __launch_bounds__(kThreads) void rms_norm_kernel(float* v, const float* w, int64_t dim, float eps) {
    rms_norm_block(v, w, v, dim, eps);
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

// The new cache row: RMSNorm of the latent part with kv_norm, RoPE of the
// positional part (one workgroup).
__global__ __launch_bounds__(kThreads) void mla_kv_row_kernel(const float* __restrict__ kvraw,
                                                             const float* __restrict__ kv_norm, float* __restrict__ kv_row,
                                                             float* __restrict__ pe_row, const float* __restrict__ cs,
                                                             const float* __restrict__ sn, int64_t R, int64_t rope,
                                                             float eps) {
    rms_norm_block(kvraw, kv_norm, kv_row, R, eps);
    if ((rope & 1) == 0) {
        for (int64_t p = threadIdx.x; p < rope / 2; p += kThreads) rope_pair(kvraw + R, pe_row, p, cs, sn);
    } else {
        for (int64_t d = threadIdx.x; d < rope; d += kThreads) pe_row[d] = kvraw[R + d];
    }
}

int gemv(const float* W, const float* x, float* y, int64_t N, int64_t K, hipStream_t st) {
    const bool vec = K % 4 == 0 && plm::aligned16(W) && plm::aligned16(x);
    const dim3 grid(static_cast<unsigned>(plm::ceil_div(N, kThreads / 64)));
    if (vec)
        hipLaunchKernelGGL(f32_gemv_kernel<true>, grid, dim3(kThreads), 0, st, W, x, y, N, K);
    else
        hipLaunchKernelGGL(f32_gemv_kernel<false>, grid, dim3(kThreads), 0, st, W, x, y, N, K);
    return plm::check_launch("f32 gemv");
}

// Query columns per chunk thread of the split kernel (its instances).
int split_cpt(int64_t R) { return R <= 4 * kChunks ? 4 : (R <= 32 * kChunks ? 32 : 64); }
int split_ppt(int64_t rope) { return rope <= 4 * kChunks ? 4 : 16; }

// Tokens per split: a multiple of 16, at most kMaxSplits splits.
int64_t tokens_per_split(int64_t L) {
    return plm::ceil_div(plm::ceil_div(L, kMaxSplits), kTileTokens) * kTileTokens;
}

size_t flash_workspace_bytes(int64_t H, int64_t L, int64_t R) {
    const int64_t nsplit = plm::ceil_div(L, tokens_per_split(L));
    return static_cast<size_t>(H * R + nsplit * H * R + nsplit * H * 2) * sizeof(float);
}

// The three MLA launches; ws holds flash_workspace_bytes.
int flash(const float* q_nope, const float* q_pe, const float* kv, const float* pe, const float* wkv_b, float* out,
          int64_t H, int64_t L, int64_t nope, int64_t rope, int64_t R, int64_t v, float scale, float* ws,
          hipStream_t st) {
    const int64_t per = tokens_per_split(L);
    const int64_t nsplit = plm::ceil_div(L, per);
    float* q_abs = ws;
    float* part = q_abs + H * R;
    float* ml = part + nsplit * H * R;
    hipLaunchKernelGGL(mla_qabs_kernel, dim3(static_cast<unsigned>(H), static_cast<unsigned>(plm::ceil_div(R, 64))),
                       dim3(kThreads), 0, st, q_nope, wkv_b, q_abs, nope, R, v);
    int code = plm::check_launch("mla q_abs kernel");
    if (code != 0) return code;
    const dim3 sgrid(static_cast<unsigned>(nsplit), static_cast<unsigned>(plm::ceil_div(H, kHeadsPerGroup)));
    // q_pe / pe are not read when rope is 0 (the reference still requires them)
#define PLM_MLA_SPLIT(C, P)                                                                                    \
    hipLaunchKernelGGL((mla_split_kernel<C, P>), sgrid, dim3(kThreads), split_lds_bytes(C, P), st, q_abs, q_pe, kv, \
                       pe, part, ml, H, L, R, rope, scale, per)
    const int cpt = split_cpt(R), ppt = split_ppt(rope);
    if (cpt == 4 && ppt == 4)
        PLM_MLA_SPLIT(4, 4);
    else if (cpt == 32 && ppt == 4)
        PLM_MLA_SPLIT(32, 4);
    else if (cpt == 32 && ppt == 16)
        PLM_MLA_SPLIT(32, 16);
    else if (cpt == 4 && ppt == 16)
        PLM_MLA_SPLIT(4, 16);
    else if (cpt == 64 && ppt == 4)
        PLM_MLA_SPLIT(64, 4);
    else
        PLM_MLA_SPLIT(64, 16);
#undef PLM_MLA_SPLIT
    code = plm::check_launch("mla split kernel");
    if (code != 0) return code;
    hipLaunchKernelGGL(mla_merge_out_kernel, dim3(static_cast<unsigned>(H), static_cast<unsigned>(plm::ceil_div(v, 32))),
                       dim3(kThreads), static_cast<size_t>(R) * sizeof(float), st, part, ml, wkv_b, out, H, nsplit,
                       nope, R, v);
    return plm::check_launch("mla merge kernel");
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
    const int64_t H = num_heads, nope = qk_nope_dim, rope = qk_rope_dim, R = kv_lora_rank, v = v_head_dim;
    const int64_t qw = nope + rope, L = previous_len + 1;
    hipStream_t st = plm::current_stream();
    // scratch: q_low, q, q_nope, q_pe, kvraw, heads, then the flash workspace
    const int64_t scratch = q_lora_rank + H * qw + H * nope + H * rope + (R + rope) + H * v;
    const int64_t pad = (scratch + 63) & ~int64_t(63);
    float* ws = static_cast<float*>(
        plm::workspace(static_cast<size_t>(pad) * sizeof(float) + flash_workspace_bytes(H, L, R)));
    if (ws == nullptr) return -3;
    float* q_low = ws;
    float* q = q_low + q_lora_rank;
    float* qn = q + H * qw;
    float* qp = qn + H * nope;
    float* kvraw = qp + H * rope;
    float* heads = kvraw + R + rope;
    float* fws = ws + pad;

    int code = gemv(q_a_weight, hidden_in, q_low, q_lora_rank, hidden_dim, st);
    if (code != 0) return code;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(kThreads), 0, st, q_low, q_norm_weight, q_lora_rank, rms_eps);
    if ((code = plm::check_launch("rms norm")) != 0) return code;
    if ((code = gemv(q_b_weight, q_low, q, H * qw, q_lora_rank, st)) != 0) return code;
    const int64_t qn_threads = std::max(H * nope, H * rope);
    hipLaunchKernelGGL(mla_q_split_kernel, dim3(static_cast<unsigned>(plm::ceil_div(std::max<int64_t>(qn_threads, 1), kThreads))),
                       dim3(kThreads), 0, st, q, qn, qp, rope_cos, rope_sin, H, nope, rope);
    if ((code = plm::check_launch("mla q split")) != 0) return code;
    // the previous rows, then the new one (ds_forward.cpp:716-744)
    if (previous_len > 0) {
        hipError_t err = hipSuccess;
        if (next_kv_cache != previous_kv_cache)
            err = hipMemcpyAsync(next_kv_cache, previous_kv_cache,
                                 static_cast<size_t>(previous_len * R) * sizeof(float), hipMemcpyDeviceToDevice, st);
        if (err == hipSuccess && rope > 0 && next_pe_cache != previous_pe_cache)
            err = hipMemcpyAsync(next_pe_cache, previous_pe_cache,
                                 static_cast<size_t>(previous_len * rope) * sizeof(float), hipMemcpyDeviceToDevice, st);
        if (err != hipSuccess) return plm::hip_fail(err, "previous cache copy");
    }
    if ((code = gemv(kv_a_weight, hidden_in, kvraw, R + rope, hidden_dim, st)) != 0) return code;
    hipLaunchKernelGGL(mla_kv_row_kernel, dim3(1), dim3(kThreads), 0, st, kvraw, kv_norm_weight,
                       next_kv_cache + previous_len * R, next_pe_cache + previous_len * rope, rope_cos, rope_sin, R,
                       rope, rms_eps);
    if ((code = plm::check_launch("mla kv row")) != 0) return code;
    code = flash(qn, qp, next_kv_cache, next_pe_cache, kv_b_weight, heads, H, L, nope, rope, R, v, softmax_scale, fws,
                 st);
    if (code != 0) return code > 0 ? 100 + code : code;
    if ((code = gemv(o_weight, heads, hidden_out, hidden_dim, H * v, st)) != 0) return code;
    return plm_ds_session_note_fused_attention(handle);
}
