// Dense decoder layer decode with a device-resident KV cache
// (src/pcketlm/native/fp16_kv_cache.cpp: the session 12-46 and 594-778, the
// attention decode 920-1060, the layer 1398-1531 and its row8-packed entry
// 1533-1589).
//
// Cache layout: one allocation per session, [layer][K|V][max_seq_len][kv_width]
// fp16/bf16.  The reference keeps committed and tentative rows in separate
// vectors; here they sit back to back in token order (committed rows, then
// tentative rows), so commit and rollback only move the two lengths (kept on
// the host) and attention reads one contiguous run of rows.
//
// One decode step is a sequence of launches on the caller's stream:
//   row8 GEMV              input RMSNorm (rounded to the storage type), then
//                          q, k, v (+ biases), in one launch
//   qk_rope_append_kernel  per-head q/k RMSNorm, RoPE, k/v rounded into the cache
//   attention_split_kernel flash-decode partials over (kv head, token split)
//   attention_merge_kernel partials -> context (fp32)
//   row8 GEMV              o projection from the fp32 context
//   post_attention_kernel  residual add, post RMSNorm
//   row8 GEMV              gate and up in one launch
//   row8 GEMV              down projection of silu(gate) * up, plus the
//                          residual, rounded to the storage type
// The weights dominate the bytes (466 MB for a Qwen2.5-7B layer); everything
// else reads or writes a few hundred KB.
#include <algorithm>
#include <cmath>
#include <vector>

#include "row8.h"

namespace {

constexpr int kNormThreads = 1024;
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / plm::kWave;
constexpr int kMaxGroup = 16;     // query heads per kv head
constexpr int kMaxHeadDim = 256;
constexpr int kMaxSplitLen = 256; // tokens per attention workgroup
constexpr int kTokUnroll = 4;      // tokens whose loads a wave issues together
constexpr int kMergeThreads = 1024;
constexpr int kMaxSplits = 4096;   // splits per head the merge stages in LDS

__device__ __forceinline__ float rd16(uint16_t v, bool bf16) {
    if (bf16) return __uint_as_float(static_cast<uint32_t>(v) << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// fp32 -> storage type: fp16 round-to-nearest-even (F16C imm 0), bf16 by
// adding 0x7FFF + lsb (fp16_kv_cache.cpp:56-75; no NaN special case).
__device__ __forceinline__ uint16_t wr16(float v, bool bf16) {
    if (bf16) {
        const uint32_t bits = __float_as_uint(v);
        return static_cast<uint16_t>((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
    }
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

__device__ __forceinline__ float wave_sum_all(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max_all(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Sum over the workgroup (kNormThreads threads), returned to every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum_all(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    const int nw = blockDim.x >> 6;
    for (int w = 0; w < nw; ++w) t += red[w];
    __syncthreads();
    return t;
}

// Per-head q/k RMSNorm (rms_norm_heads_inplace, 561-584), RoPE at `pos`
// (apply_rope_one, 518-539), q kept in fp32, k and v rounded into cache row
// `pos`.  One wave per head: blocks [0, nh) take q heads, [nh, nh + nkv) k/v.
template <bool BF16>
__global__ __launch_bounds__(64) void qk_rope_append_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v,
                                                            const uint16_t* __restrict__ q_norm,
                                                            const uint16_t* __restrict__ k_norm,
                                                            float* __restrict__ q_rot, uint16_t* __restrict__ k_row,
                                                            uint16_t* __restrict__ v_row, int nh, int hd, int64_t pos,
                                                            float theta, float eps) {
#pragma clang fp contract(off)
    const int head = blockIdx.x;
    const int lane = threadIdx.x;
    const bool is_q = head < nh;
    const int kvh = head - nh;
    const float* src = is_q ? q + static_cast<int64_t>(head) * hd : k + static_cast<int64_t>(kvh) * hd;
    const uint16_t* nw = is_q ? q_norm : k_norm;
    float scale = 1.0f;
    if (nw != nullptr) {
        float s = 0.0f;
        for (int d = lane; d < hd; d += 64) s += src[d] * src[d];
        const float ms = wave_sum_all(s) / static_cast<float>(hd);
        scale = 1.0f / sqrtf(ms + eps);
    }
    const int half = hd / 2;
    for (int p = lane; p < half; p += 64) {
        float x0 = src[p], x1 = src[p + half];
        if (nw != nullptr) {
            x0 = x0 * scale * rd16(nw[p], BF16);
            x1 = x1 * scale * rd16(nw[p + half], BF16);
        }
        const float inv_freq = powf(theta, -(2.0f * static_cast<float>(p)) / static_cast<float>(hd));
        const float angle = static_cast<float>(pos) * inv_freq;
        const float c = cosf(angle), sn = sinf(angle);
        const float y0 = x0 * c - x1 * sn;
        const float y1 = x1 * c + x0 * sn;
        if (is_q) {
            q_rot[static_cast<int64_t>(head) * hd + p] = y0;
            q_rot[static_cast<int64_t>(head) * hd + p + half] = y1;
        } else {
            k_row[static_cast<int64_t>(kvh) * hd + p] = wr16(y0, BF16);
            k_row[static_cast<int64_t>(kvh) * hd + p + half] = wr16(y1, BF16);
        }
    }
    if ((hd & 1) != 0 && lane == 0) {  // an odd head keeps its last element unrotated
        float x = src[hd - 1];
        if (nw != nullptr) x = x * scale * rd16(nw[hd - 1], BF16);
        if (is_q) {
            q_rot[static_cast<int64_t>(head) * hd + hd - 1] = x;
        } else {
            k_row[static_cast<int64_t>(kvh) * hd + hd - 1] = wr16(x, BF16);
        }
    }
    if (!is_q)
        for (int d = lane; d < hd; d += 64)
            v_row[static_cast<int64_t>(kvh) * hd + d] = wr16(v[static_cast<int64_t>(kvh) * hd + d], BF16);
}

// Flash-decode partials.  Block (kvh, sp) takes tokens [sp*L, min(T, sp*L+L))
// of kv head kvh for its `group` query heads: scores q.k * scale into LDS,
// per-head max m and sum l of exp(score - m), and acc = sum exp(score - m) v.
// Waves take tokens, lanes take head dimensions.
// G bounds the query heads per kv head (group <= G), DPL the head dimensions
// per lane (hd <= 64 * DPL): the unrolled body stays small enough for the
// instruction cache.
template <bool BF16, int G, int DPL>
__global__ __launch_bounds__(kAttnThreads) void attention_split_kernel(
    const float* __restrict__ q_rot, const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    int64_t kv_width, int hd, int group, int64_t T, int L, float scale, float* __restrict__ part,
    float* __restrict__ ml) {
    extern __shared__ float sm[];
    float* q_s = sm;                   // [group][hd], later the cross-wave sum
    float* p_s = sm + group * hd;      // [group][L]
    const int kvh = blockIdx.x, sp = blockIdx.y, nsplit = gridDim.y;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t t0 = static_cast<int64_t>(sp) * L;
    const int n = static_cast<int>(min(static_cast<int64_t>(L), T - t0));
    for (int i = threadIdx.x; i < group * hd; i += kAttnThreads)
        q_s[i] = q_rot[static_cast<int64_t>(kvh) * group * hd + i];
    __syncthreads();

    // Scores: a wave loads the rows of kTokUnroll tokens before using any;
    // the V rows of its first tokens are loaded at the same time (vpre) so
    // that the value pass does not start with a full memory latency.
    float vpre[kTokUnroll][DPL];
    for (int i0 = wave; i0 < n; i0 += kAttnWaves * kTokUnroll) {
        float kv[kTokUnroll][DPL];
#pragma unroll
        for (int u = 0; u < kTokUnroll; ++u) {
            const int i = min(i0 + u * kAttnWaves, n - 1);
            const uint16_t* kr = k_cache + (t0 + i) * kv_width + static_cast<int64_t>(kvh) * hd;
            const uint16_t* vr = v_cache + (t0 + i) * kv_width + static_cast<int64_t>(kvh) * hd;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                const int d = lane + 64 * j;
                kv[u][j] = d < hd ? rd16(kr[d], BF16) : 0.0f;
                if (i0 == wave) vpre[u][j] = d < hd ? rd16(vr[d], BF16) : 0.0f;
            }
        }
#pragma unroll
        for (int u = 0; u < kTokUnroll; ++u) {
            const int i = i0 + u * kAttnWaves;
            if (i >= n) break;
            float acc[G];
#pragma unroll
            for (int h = 0; h < G; ++h) acc[h] = 0.0f;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                const int d = lane + 64 * j;
                if (d < hd) {
#pragma unroll
                    for (int h = 0; h < G; ++h)
                        if (h < group) acc[h] = fmaf(q_s[h * hd + d], kv[u][j], acc[h]);
                }
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                if (h < group) {
                    const float sum = plm_wave_sum(acc[h]);
                    if (lane == kSumLane) p_s[h * L + i] = sum * scale;
                }
            }
        }
    }
    __syncthreads();

    for (int h = wave; h < group; h += kAttnWaves) {
        float m = -INFINITY;
        for (int i = lane; i < n; i += 64) m = fmaxf(m, p_s[h * L + i]);
        m = wave_max_all(m);
        float l = 0.0f;
        for (int i = lane; i < n; i += 64) {
            const float e = expf(p_s[h * L + i] - m);
            p_s[h * L + i] = e;
            l += e;
        }
        l = wave_sum_all(l);
        if (lane == 0) {
            const int64_t slot = (static_cast<int64_t>(kvh) * nsplit + sp) * group + h;
            ml[slot * 2] = m;
            ml[slot * 2 + 1] = l;
        }
    }
    __syncthreads();

    float acc[G][DPL];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[h][j] = 0.0f;
    for (int i0 = wave; i0 < n; i0 += kAttnWaves * kTokUnroll) {
        float vv[kTokUnroll][DPL];
#pragma unroll
        for (int u = 0; u < kTokUnroll; ++u) {
            const int i = min(i0 + u * kAttnWaves, n - 1);
            const uint16_t* vr = v_cache + (t0 + i) * kv_width + static_cast<int64_t>(kvh) * hd;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                const int d = lane + 64 * j;
                vv[u][j] = i0 == wave ? vpre[u][j] : (d < hd ? rd16(vr[d], BF16) : 0.0f);
            }
        }
#pragma unroll
        for (int u = 0; u < kTokUnroll; ++u) {
            const int i = i0 + u * kAttnWaves;
            if (i >= n) break;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                if (lane + 64 * j < hd) {
#pragma unroll
                    for (int h = 0; h < G; ++h)
                        if (h < group) acc[h][j] = fmaf(p_s[h * L + i], vv[u][j], acc[h][j]);
                }
            }
        }
    }
    // Waves add their sums into q_s (free again) one after another.
    for (int w = 0; w < kAttnWaves; ++w) {
        if (wave == w) {
#pragma unroll
            for (int h = 0; h < G; ++h) {
#pragma unroll
                for (int j = 0; j < DPL; ++j) {
                    const int d = lane + 64 * j;
                    if (h < group && d < hd) q_s[h * hd + d] = (w == 0 ? 0.0f : q_s[h * hd + d]) + acc[h][j];
                }
            }
        }
        __syncthreads();
    }
    float* dst = part + (static_cast<int64_t>(kvh) * nsplit + sp) * group * hd;
    for (int i = threadIdx.x; i < group * hd; i += kAttnThreads) dst[i] = q_s[i];
}

template <bool BF16, int G>
void launch_split_g(int dpl, dim3 grid, size_t lds, hipStream_t st, const float* q_rot, const uint16_t* kc,
                    const uint16_t* vc, int64_t kvw, int hd, int group, int64_t T, int L, float scale, float* part,
                    float* ml) {
    if (dpl <= 1) {
        hipLaunchKernelGGL((attention_split_kernel<BF16, G, 1>), grid, dim3(kAttnThreads), lds, st, q_rot, kc, vc, kvw,
                           hd, group, T, L, scale, part, ml);
    } else if (dpl == 2) {
        hipLaunchKernelGGL((attention_split_kernel<BF16, G, 2>), grid, dim3(kAttnThreads), lds, st, q_rot, kc, vc, kvw,
                           hd, group, T, L, scale, part, ml);
    } else {
        hipLaunchKernelGGL((attention_split_kernel<BF16, G, 4>), grid, dim3(kAttnThreads), lds, st, q_rot, kc, vc, kvw,
                           hd, group, T, L, scale, part, ml);
    }
}

template <bool BF16>
void launch_split(dim3 grid, size_t lds, hipStream_t st, const float* q_rot, const uint16_t* kc, const uint16_t* vc,
                  int64_t kvw, int hd, int group, int64_t T, int L, float scale, float* part, float* ml) {
    const int dpl = (hd + 63) / 64;
    if (group <= 1) {
        launch_split_g<BF16, 1>(dpl, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, L, scale, part, ml);
    } else if (group <= 2) {
        launch_split_g<BF16, 2>(dpl, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, L, scale, part, ml);
    } else if (group <= 4) {
        launch_split_g<BF16, 4>(dpl, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, L, scale, part, ml);
    } else if (group <= 8) {
        launch_split_g<BF16, 8>(dpl, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, L, scale, part, ml);
    } else {
        launch_split_g<BF16, kMaxGroup>(dpl, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, L, scale, part, ml);
    }
}

// context[h][d] = sum_s exp(m_s - M) acc_s[d] / sum_s exp(m_s - M) l_s.
// One workgroup per query head: the split factors exp(m_s - M) go to LDS,
// then thread (c, d) sums splits c, c + C, ... of dimension d with several
// loads in flight, and the C partial sums are added in LDS.
__global__ __launch_bounds__(kMergeThreads) void attention_merge_kernel(const float* __restrict__ part,
                                                                       const float* __restrict__ ml,
                                                                       float* __restrict__ context, int hd, int group,
                                                                       int nsplit) {
    __shared__ float f_s[kMaxSplits];
    __shared__ float red[kMergeThreads / 64];
    __shared__ float sums[kMergeThreads];
    const int head = blockIdx.x;
    const int kvh = head / group, hl = head - kvh * group;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t base = static_cast<int64_t>(kvh) * nsplit * group + hl;  // slot of split s: base + s * group
    float m = -INFINITY;
    for (int sp = tid; sp < nsplit; sp += kMergeThreads) m = fmaxf(m, ml[(base + static_cast<int64_t>(sp) * group) * 2]);
    m = wave_max_all(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < kMergeThreads / 64; ++w) m = fmaxf(m, red[w]);
    __syncthreads();
    float den = 0.0f;
    for (int sp = tid; sp < nsplit; sp += kMergeThreads) {
        const int64_t slot = base + static_cast<int64_t>(sp) * group;
        const float f = expf(ml[slot * 2] - m);
        f_s[sp] = f;
        den += f * ml[slot * 2 + 1];
    }
    den = block_sum(den, red);  // its barriers also publish f_s
    const int C = kMergeThreads / hd;  // split lanes per dimension (hd <= kMergeThreads)
    const int c = tid / hd, d = tid - c * hd;
    float num = 0.0f;
    if (c < C) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        int sp = c;
        for (; sp + 3 * C < nsplit; sp += 4 * C) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t slot = base + static_cast<int64_t>(sp + u * C) * group;
                acc[u] = fmaf(f_s[sp + u * C], part[slot * hd + d], acc[u]);
            }
        }
        for (; sp < nsplit; sp += C) acc[0] = fmaf(f_s[sp], part[(base + static_cast<int64_t>(sp) * group) * hd + d], acc[0]);
        num = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    sums[tid] = num;
    __syncthreads();
    if (tid < hd) {
        float t = 0.0f;
        for (int k = 0; k < C; ++k) t += sums[k * hd + tid];
        context[static_cast<int64_t>(head) * hd + tid] = t / den;
    }
}

// attention_out = storage(proj); resid = hidden + attention_out (fp32);
// post = storage(rms_norm(storage(resid)) * w)   (1468-1491).
template <bool BF16>
__global__ __launch_bounds__(kNormThreads) void post_attention_kernel(const uint16_t* __restrict__ hidden,
                                                                      const float* __restrict__ proj,
                                                                      const uint16_t* __restrict__ w,
                                                                      float* __restrict__ resid,
                                                                      uint16_t* __restrict__ post, int n, float eps) {
#pragma clang fp contract(off)
    __shared__ float red[kNormThreads / 64];
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float r = rd16(hidden[i], BF16) + rd16(wr16(proj[i], BF16), BF16);
        resid[i] = r;
        const float rq = rd16(wr16(r, BF16), BF16);
        s += rq * rq;
    }
    const float ms = block_sum(s, red) / static_cast<float>(n);
    const float scale = 1.0f / sqrtf(ms + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        post[i] = wr16(rd16(wr16(resid[i], BF16), BF16) * scale * rd16(w[i], BF16), BF16);
}

struct LayerLengths {
    int64_t committed = 0;
    int64_t tentative = 0;
};

struct KvSession {
    int64_t layer_count = 0;
    int64_t max_seq_len = 0;
    int64_t kv_width = 0;
    int dtype_code = 0;
    int device = 0;
    uint16_t* cache = nullptr;  // [layer][2][max_seq_len][kv_width]
    std::vector<LayerLengths> layers;

    uint16_t* k_rows(int64_t layer) const { return cache + (layer * 2) * max_seq_len * kv_width; }
    uint16_t* v_rows(int64_t layer) const { return cache + (layer * 2 + 1) * max_seq_len * kv_width; }
};

bool valid_layer(const KvSession* s, int64_t layer) { return s != nullptr && layer >= 0 && layer < s->layer_count; }

size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

int copy_rows(void* dst, const void* src, size_t bytes, hipStream_t st) {
    if (bytes == 0) return 0;
    const hipError_t err = hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, st);
    return err == hipSuccess ? 0 : plm::hip_fail(err, "hipMemcpyAsync (kv cache)");
}

// append_to_region (626-659): count rows at the end of the committed or the
// tentative run.  Committed rows go in front of the tentative ones, which
// move back by `count` rows through the workspace.
int append_rows(KvSession* s, int64_t layer, const uint16_t* k_new, const uint16_t* v_new, int64_t count,
                bool tentative) {
    if (!valid_layer(s, layer) || k_new == nullptr || v_new == nullptr || count < 0) return 1;
    LayerLengths& st = s->layers[static_cast<size_t>(layer)];
    if (st.committed + st.tentative + count > s->max_seq_len) return 2;
    if (count == 0) return 0;
    const hipStream_t stream = plm::current_stream();
    const size_t row_bytes = static_cast<size_t>(s->kv_width) * 2;
    const size_t new_bytes = static_cast<size_t>(count) * row_bytes;
    uint16_t* kb = s->k_rows(layer);
    uint16_t* vb = s->v_rows(layer);
    int code = 0;
    if (tentative) {
        const int64_t at = (st.committed + st.tentative) * s->kv_width;
        code = copy_rows(kb + at, k_new, new_bytes, stream);
        if (code == 0) code = copy_rows(vb + at, v_new, new_bytes, stream);
        if (code == 0) st.tentative += count;
        return code;
    }
    const int64_t at = st.committed * s->kv_width;
    const size_t tail_bytes = static_cast<size_t>(st.tentative) * row_bytes;
    char* tmp = nullptr;
    if (tail_bytes != 0) {
        tmp = static_cast<char*>(plm::workspace(2 * tail_bytes));
        if (tmp == nullptr) return plm::fail(3, "workspace for the tentative rows");
        code = copy_rows(tmp, kb + at, tail_bytes, stream);
        if (code == 0) code = copy_rows(tmp + tail_bytes, vb + at, tail_bytes, stream);
    }
    if (code == 0) code = copy_rows(kb + at, k_new, new_bytes, stream);
    if (code == 0) code = copy_rows(vb + at, v_new, new_bytes, stream);
    if (code == 0 && tail_bytes != 0) {
        const int64_t moved = (st.committed + count) * s->kv_width;
        code = copy_rows(kb + moved, tmp, tail_bytes, stream);
        if (code == 0) code = copy_rows(vb + moved, tmp + tail_bytes, tail_bytes, stream);
    }
    if (code == 0) st.committed += count;
    return code;
}

struct DenseArgs {
    const uint16_t *hidden, *input_norm, *post_norm;
    const uint16_t *q_w, *k_w, *v_w, *o_w, *gate_w, *up_w, *down_w;
    const uint16_t *q_bias, *k_bias, *v_bias, *q_norm, *k_norm;
    uint16_t* out;
    int64_t hidden_size, inter, nh, nkv;
    float eps, theta;
};

// Attention split length: about eight workgroups per CU over (kv head, split),
// at least 16 tokens each, at most kMaxSplitLen.
int split_len_for(int64_t T, int64_t nkv) {
    const int64_t target = std::max<int64_t>(1, 8 * plm::cu_count() / std::max<int64_t>(1, nkv));
    int64_t L = (T + target - 1) / target;
    L = ((L + 15) / 16) * 16;
    return static_cast<int>(std::min<int64_t>(std::max<int64_t>(L, 16), kMaxSplitLen));
}

template <bool BF16>
int dense_decode(KvSession* s, int64_t layer, const DenseArgs& a) {
    // Attention-stage checks keep the reference's codes, offset by 100.
    if (!valid_layer(s, layer)) return 101;
    if (a.nh <= 0 || a.nkv <= 0) return 102;
    if (a.hidden_size % a.nh != 0 || a.nh % a.nkv != 0) return 103;
    const int64_t hd = a.hidden_size / a.nh;
    const int64_t kvw = a.nkv * hd;
    if (kvw != s->kv_width) return 104;
    LayerLengths& st = s->layers[static_cast<size_t>(layer)];
    const int64_t pos = st.committed + st.tentative;
    if (pos + 1 > s->max_seq_len) return 105;
    const int64_t group = a.nh / a.nkv;
    if (group > kMaxGroup || hd > kMaxHeadDim)
        return plm::fail(106, "head shape outside the kernels' limits (%lld query heads per kv head, head_dim %lld)",
                         static_cast<long long>(group), static_cast<long long>(hd));
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev != s->device) return plm::fail(107, "session lives on another device");

    const int64_t H = a.hidden_size, I = a.inter, T = pos + 1;
    const int L = split_len_for(T, a.nkv);
    const int64_t nsplit = (T + L - 1) / L;
    if (nsplit > kMaxSplits) return plm::fail(106, "context too long for one attention launch");
    // workspace: q f32[H] | k, v f32[kvw] | q_rot f32[H] | part | ml | ctx f32[H] | proj f32[H] | resid f32[H]
    //            | post u16[H] | gate, up f32[I]
    const size_t sz[] = {static_cast<size_t>(H) * 4, static_cast<size_t>(kvw) * 4, static_cast<size_t>(kvw) * 4,
                         static_cast<size_t>(H) * 4, static_cast<size_t>(a.nh * nsplit * hd) * 4,
                         static_cast<size_t>(a.nh * nsplit) * 8, static_cast<size_t>(H) * 4,
                         static_cast<size_t>(H) * 4, static_cast<size_t>(H) * 4, static_cast<size_t>(H) * 2,
                         static_cast<size_t>(I) * 4, static_cast<size_t>(I) * 4};
    constexpr int nbuf = static_cast<int>(sizeof(sz) / sizeof(sz[0]));
    size_t off[nbuf];
    size_t total = 0;
    for (int i = 0; i < nbuf; ++i) {
        off[i] = total;
        total += align256(sz[i]);
    }
    char* ws = static_cast<char*>(plm::workspace(total));
    if (ws == nullptr) return plm::fail(108, "workspace");
    float* q = reinterpret_cast<float*>(ws + off[0]);
    float* k = reinterpret_cast<float*>(ws + off[1]);
    float* v = reinterpret_cast<float*>(ws + off[2]);
    float* q_rot = reinterpret_cast<float*>(ws + off[3]);
    float* part = reinterpret_cast<float*>(ws + off[4]);
    float* ml = reinterpret_cast<float*>(ws + off[5]);
    float* ctx = reinterpret_cast<float*>(ws + off[6]);
    float* proj = reinterpret_cast<float*>(ws + off[7]);
    float* resid = reinterpret_cast<float*>(ws + off[8]);
    uint16_t* post = reinterpret_cast<uint16_t*>(ws + off[9]);
    float* gate = reinterpret_cast<float*>(ws + off[10]);
    float* up = reinterpret_cast<float*>(ws + off[11]);
    const hipStream_t stream = plm::current_stream();
    const int dc = BF16 ? 1 : 0;
    int code = 0;

    plm::Row8X x_in;  // the input RMSNorm is the q/k/v launch's prologue
    x_in.u16 = a.hidden;
    x_in.norm_w = a.input_norm;
    x_in.eps = a.eps;
    plm::Row8Mat qkv[3] = {{a.q_w, a.q_bias, q, H}, {a.k_w, a.k_bias, k, kvw}, {a.v_w, a.v_bias, v, kvw}};
    if ((code = plm::row8_gemv_x(x_in, qkv, 3, H, dc, stream)) != 0) return code;
    uint16_t* k_row = s->k_rows(layer) + pos * kvw;
    uint16_t* v_row = s->v_rows(layer) + pos * kvw;
    hipLaunchKernelGGL((qk_rope_append_kernel<BF16>), dim3(static_cast<unsigned>(a.nh + a.nkv)), dim3(64), 0, stream,
                       q, k, v, a.q_norm, a.k_norm, q_rot, k_row, v_row, static_cast<int>(a.nh), static_cast<int>(hd),
                       pos, a.theta, a.eps);
    if ((code = plm::check_launch("q/k rope and cache append")) != 0) return code;
    st.tentative += 1;  // the row is in the cache once the stream reaches here

    const size_t lds = static_cast<size_t>(group) * (hd + L) * sizeof(float);
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    launch_split<BF16>(dim3(static_cast<unsigned>(a.nkv), static_cast<unsigned>(nsplit)), lds, stream, q_rot,
                       s->k_rows(layer), s->v_rows(layer), kvw, static_cast<int>(hd), static_cast<int>(group), T, L,
                       scale, part, ml);
    if ((code = plm::check_launch("attention split")) != 0) return code;
    hipLaunchKernelGGL(attention_merge_kernel, dim3(static_cast<unsigned>(a.nh)), dim3(kMergeThreads), 0, stream,
                       part, ml, ctx,
                       static_cast<int>(hd), static_cast<int>(group), static_cast<int>(nsplit));
    if ((code = plm::check_launch("attention merge")) != 0) return code;
    plm::Row8Mat o = {a.o_w, nullptr, proj, H};
    if ((code = plm::row8_gemv(nullptr, ctx, &o, 1, H, dc, stream)) != 0) return code;
    hipLaunchKernelGGL((post_attention_kernel<BF16>), dim3(1), dim3(kNormThreads), 0, stream, a.hidden, proj,
                       a.post_norm, resid, post, static_cast<int>(H), a.eps);
    if ((code = plm::check_launch("post attention norm")) != 0) return code;
    plm::Row8Mat gu[2] = {{a.gate_w, nullptr, gate, I}, {a.up_w, nullptr, up, I}};
    if ((code = plm::row8_gemv(post, nullptr, gu, 2, H, dc, stream)) != 0) return code;
    plm::Row8X x_act;  // SiLU(gate) * up is read by the down launch, which adds the residual
    x_act.f32 = gate;
    x_act.f32_b = up;
    plm::Row8Mat down = {a.down_w, nullptr, nullptr, H, 0, resid, a.out};
    return plm::row8_gemv_x(x_act, &down, 1, I, dc, stream);
}

}  // namespace

// ====================================================================== C ABI

PLM_EXPORT void* kv_prefill_init_typed(int64_t layer_count, int64_t max_seq_len, int64_t kv_width, int dtype_code) {
    plm::clear_error();
    if (layer_count <= 0 || max_seq_len <= 0 || kv_width <= 0 || (dtype_code != 0 && dtype_code != 1)) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    const size_t bytes = static_cast<size_t>(layer_count) * 2 * static_cast<size_t>(max_seq_len) *
                         static_cast<size_t>(kv_width) * sizeof(uint16_t);
    void* cache = nullptr;
    const hipError_t err = hipMalloc(&cache, bytes);
    if (err != hipSuccess) {
        plm::hip_fail(err, "hipMalloc(kv cache)");
        return nullptr;
    }
    KvSession* s = new KvSession();
    s->layer_count = layer_count;
    s->max_seq_len = max_seq_len;
    s->kv_width = kv_width;
    s->dtype_code = dtype_code;
    s->device = dev;
    s->cache = static_cast<uint16_t*>(cache);
    s->layers.resize(static_cast<size_t>(layer_count));
    return s;
}

PLM_EXPORT void* kv_prefill_init(int64_t layer_count, int64_t max_seq_len, int64_t kv_width) {
    return kv_prefill_init_typed(layer_count, max_seq_len, kv_width, 0);
}

PLM_EXPORT void kv_free(void* handle) {
    KvSession* s = static_cast<KvSession*>(handle);
    if (s == nullptr) return;
    if (s->cache != nullptr) {
        (void)hipDeviceSynchronize();  // kernels of earlier calls may still read the rows
        (void)hipFree(s->cache);
    }
    delete s;
}

PLM_EXPORT int kv_append_committed(void* handle, int64_t layer, const uint16_t* k_new, const uint16_t* v_new,
                                   int64_t count) {
    plm::clear_error();
    return append_rows(static_cast<KvSession*>(handle), layer, k_new, v_new, count, false);
}

PLM_EXPORT int kv_append_tentative(void* handle, int64_t layer, const uint16_t* k_new, const uint16_t* v_new,
                                   int64_t count) {
    plm::clear_error();
    return append_rows(static_cast<KvSession*>(handle), layer, k_new, v_new, count, true);
}

PLM_EXPORT int kv_commit(void* handle, int64_t count) {
    KvSession* s = static_cast<KvSession*>(handle);
    if (s == nullptr || count < 0) return 1;
    for (LayerLengths& st : s->layers) {
        const int64_t take = std::min(count, st.tentative);
        st.committed += take;
        st.tentative -= take;
    }
    return 0;
}

PLM_EXPORT int kv_rollback(void* handle) {
    KvSession* s = static_cast<KvSession*>(handle);
    if (s == nullptr) return 1;
    for (LayerLengths& st : s->layers) st.tentative = 0;
    return 0;
}

PLM_EXPORT int64_t kv_committed_length(void* handle, int64_t layer) {
    const KvSession* s = static_cast<const KvSession*>(handle);
    return valid_layer(s, layer) ? s->layers[static_cast<size_t>(layer)].committed : -1;
}

PLM_EXPORT int64_t kv_tentative_length(void* handle, int64_t layer) {
    const KvSession* s = static_cast<const KvSession*>(handle);
    return valid_layer(s, layer) ? s->layers[static_cast<size_t>(layer)].tentative : -1;
}

PLM_EXPORT int kv_copy_layer(void* handle, int64_t layer, uint16_t* k_out, uint16_t* v_out, int64_t max_count,
                             int include_tentative) {
    plm::clear_error();
    KvSession* s = static_cast<KvSession*>(handle);
    if (!valid_layer(s, layer) || k_out == nullptr || v_out == nullptr || max_count < 0) return 1;
    const LayerLengths& st = s->layers[static_cast<size_t>(layer)];
    const int64_t rows = st.committed + (include_tentative ? st.tentative : 0);
    if (rows > max_count) return 2;
    const size_t bytes = static_cast<size_t>(rows * s->kv_width) * 2;
    const hipStream_t stream = plm::current_stream();
    int code = copy_rows(k_out, s->k_rows(layer), bytes, stream);
    if (code == 0) code = copy_rows(v_out, s->v_rows(layer), bytes, stream);
    return code;
}

namespace {

// The row-major (unpacked) entry points: the reference's argument checks,
// then "not implemented" (code 90).
int rowmajor_unsupported(const char* name) {
    return plm::fail(90, "%s: row-major weights are not supported by this library; pack each weight once with "
                         "native_pack_u16_rows8 and call kv_dense_layer_decode_u16_ext_packed_rows8", name);
}

}  // namespace

PLM_EXPORT int kv_attention_decode_fp16(void* handle, int64_t layer, const uint16_t* hidden, const uint16_t* q_weight,
                                        const uint16_t* k_weight, const uint16_t* v_weight, const uint16_t* o_weight,
                                        uint16_t* out, int64_t hidden_size, int64_t num_attention_heads,
                                        int64_t num_key_value_heads, float rope_theta) {
    (void)rope_theta;
    plm::clear_error();
    if (!valid_layer(static_cast<KvSession*>(handle), layer) || !hidden || !q_weight || !k_weight || !v_weight ||
        !o_weight || !out)
        return 1;
    if (hidden_size <= 0 || num_attention_heads <= 0 || num_key_value_heads <= 0) return 2;
    return rowmajor_unsupported("kv_attention_decode_fp16");
}

PLM_EXPORT int kv_attention_decode_u16_ext(void* handle, int64_t layer, const uint16_t* hidden,
                                           const uint16_t* q_weight, const uint16_t* k_weight,
                                           const uint16_t* v_weight, const uint16_t* o_weight, const uint16_t* q_bias,
                                           const uint16_t* k_bias, const uint16_t* v_bias,
                                           const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
                                           uint16_t* out, int64_t hidden_size, int64_t num_attention_heads,
                                           int64_t num_key_value_heads, float rope_theta, float rms_eps) {
    (void)q_bias, (void)k_bias, (void)v_bias, (void)q_norm_weight, (void)k_norm_weight, (void)rope_theta,
        (void)rms_eps;
    plm::clear_error();
    if (!valid_layer(static_cast<KvSession*>(handle), layer) || !hidden || !q_weight || !k_weight || !v_weight ||
        !o_weight || !out)
        return 1;
    if (hidden_size <= 0 || num_attention_heads <= 0 || num_key_value_heads <= 0) return 2;
    return rowmajor_unsupported("kv_attention_decode_u16_ext");
}

PLM_EXPORT int kv_dense_layer_decode_fp16(void* handle, int64_t layer, const uint16_t* hidden,
                                          const uint16_t* input_norm_weight, const uint16_t* post_norm_weight,
                                          const uint16_t* q_weight, const uint16_t* k_weight,
                                          const uint16_t* v_weight, const uint16_t* o_weight,
                                          const uint16_t* gate_weight, const uint16_t* up_weight,
                                          const uint16_t* down_weight, uint16_t* out, int64_t hidden_size,
                                          int64_t intermediate_size, int64_t num_heads, int64_t num_kv_heads,
                                          float rms_eps, float rope_theta) {
    (void)layer, (void)num_heads, (void)num_kv_heads, (void)rms_eps, (void)rope_theta;
    plm::clear_error();
    if (handle == nullptr || !hidden || !input_norm_weight || !post_norm_weight || !q_weight || !k_weight ||
        !v_weight || !o_weight || !gate_weight || !up_weight || !down_weight || !out)
        return 1;
    if (hidden_size <= 0 || intermediate_size <= 0) return 2;
    return rowmajor_unsupported("kv_dense_layer_decode_fp16");
}

PLM_EXPORT int kv_dense_layer_decode_u16_ext(
    void* handle, int64_t layer, const uint16_t* hidden, const uint16_t* input_norm_weight,
    const uint16_t* post_norm_weight, const uint16_t* q_weight, const uint16_t* k_weight, const uint16_t* v_weight,
    const uint16_t* o_weight, const uint16_t* gate_weight, const uint16_t* up_weight, const uint16_t* down_weight,
    const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias, const uint16_t* q_norm_weight,
    const uint16_t* k_norm_weight, uint16_t* out, int64_t hidden_size, int64_t intermediate_size, int64_t num_heads,
    int64_t num_kv_heads, float rms_eps, float rope_theta) {
    (void)layer, (void)q_bias, (void)k_bias, (void)v_bias, (void)q_norm_weight, (void)k_norm_weight, (void)num_heads,
        (void)num_kv_heads, (void)rms_eps, (void)rope_theta;
    plm::clear_error();
    if (handle == nullptr || !hidden || !input_norm_weight || !post_norm_weight || !q_weight || !k_weight ||
        !v_weight || !o_weight || !gate_weight || !up_weight || !down_weight || !out)
        return 1;
    if (hidden_size <= 0 || intermediate_size <= 0) return 2;
    return rowmajor_unsupported("kv_dense_layer_decode_u16_ext");
}

PLM_EXPORT int kv_dense_layer_decode_u16_ext_packed_rows8(
    void* handle, int64_t layer, const uint16_t* hidden, const uint16_t* input_norm_weight,
    const uint16_t* post_norm_weight, const uint16_t* q_weight_packed, const uint16_t* k_weight_packed,
    const uint16_t* v_weight_packed, const uint16_t* o_weight_packed, const uint16_t* gate_weight_packed,
    const uint16_t* up_weight_packed, const uint16_t* down_weight_packed, const uint16_t* q_bias,
    const uint16_t* k_bias, const uint16_t* v_bias, const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
    uint16_t* out, int64_t hidden_size, int64_t intermediate_size, int64_t num_heads, int64_t num_kv_heads,
    float rms_eps, float rope_theta) {
    plm::clear_error();
    if (handle == nullptr || hidden == nullptr || input_norm_weight == nullptr || post_norm_weight == nullptr ||
        q_weight_packed == nullptr || k_weight_packed == nullptr || v_weight_packed == nullptr ||
        o_weight_packed == nullptr || gate_weight_packed == nullptr || up_weight_packed == nullptr ||
        down_weight_packed == nullptr || out == nullptr)
        return 1;
    if (hidden_size <= 0 || intermediate_size <= 0) return 2;
    if (hidden_size > 0x7FFFFFFF || intermediate_size > 0x7FFFFFFF) return plm::fail(2, "dimension too large");
    KvSession* s = static_cast<KvSession*>(handle);
    const DenseArgs a = {hidden,          input_norm_weight, post_norm_weight,  q_weight_packed, k_weight_packed,
                         v_weight_packed, o_weight_packed,   gate_weight_packed, up_weight_packed, down_weight_packed,
                         q_bias,          k_bias,            v_bias,            q_norm_weight,   k_norm_weight,
                         out,             hidden_size,       intermediate_size, num_heads,       num_kv_heads,
                         rms_eps,         rope_theta};
    return s->dtype_code == 1 ? dense_decode<true>(s, layer, a) : dense_decode<false>(s, layer, a);
}
