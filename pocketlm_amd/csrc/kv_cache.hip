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
constexpr int kMergeThreads = 1024;
constexpr int kMaxSplits = 65535;  // the split launch's grid height

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

// A DPP lane swap within each 16-lane row (xor 1, xor 2, half-row mirror,
// row mirror), and one row's value read from its first lane: the pieces of
// the score and softmax reductions, with no LDS round trips.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float rows_f32(float v, int row) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * row));
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

// Flash-decode partials.  Workgroup (kvh, sp) takes the TOK tokens
// [sp * TOK, ...) of kv head kvh for its `group` query heads and writes, per
// head, the partial sum acc = sum_t exp(s_t - m) v_t, the max m of its scores
// s_t = (q . k_t) * scale and l = sum_t exp(s_t - m).
//   scores: lanes form groups of HS = min(G, 4) head slices times four
//           quarters of the head dimensions (16-byte K loads; adjacent lanes
//           read adjacent bytes); a lane dots its quarter of TPL tokens with
//           the heads of its slice, reading each query piece once for all of
//           them, then two lane swaps add the quarters;
//   softmax: TOK lanes per head, 256 / TOK heads at a time;
//   values: waves take every fourth token, lanes take VD adjacent head
//           dimensions (V rows read 64 lanes wide), accumulating all heads;
//   the four waves' sums meet in LDS behind one barrier and every thread
//   adds ((w0 + w2) + (w1 + w3)) for a few outputs.
// G bounds the query heads per kv head (group <= G), VD the head dimensions
// per lane in the value pass (hd <= 64 * VD).  TOK (16, 32 or 64) is chosen
// per launch so that short contexts still spread over the CUs.
constexpr int kMaxSplitTokens = 64;
constexpr int kMinSplitTokens = 16;
constexpr int kAttnTargetGroups = 1024;  // four workgroups per CU of an MI355X

// Max / sum over aligned segments of W lanes (16, 32 or 64), the result in
// every lane of the segment: DPP swaps within each 16-lane row, then the
// rows' results read from lanes 0, 16, 32 and 48.
template <int W>
__device__ __forceinline__ float seg_max(float v, int lane) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    if constexpr (W == 16) return v;
    const float r0 = rows_f32(v, 0), r1 = rows_f32(v, 1), r2 = rows_f32(v, 2), r3 = rows_f32(v, 3);
    if constexpr (W == 32) return lane < 32 ? fmaxf(r0, r1) : fmaxf(r2, r3);
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}
template <int W>
__device__ __forceinline__ float seg_sum(float v, int lane) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    if constexpr (W == 16) return v;
    const float r0 = rows_f32(v, 0), r1 = rows_f32(v, 1), r2 = rows_f32(v, 2), r3 = rows_f32(v, 3);
    if constexpr (W == 32) return lane < 32 ? r0 + r1 : r2 + r3;
    return (r0 + r1) + (r2 + r3);
}

// VD adjacent 16-bit values as raw words (one 32-bit word per two values),
// loaded with one instruction when vec, else value by value (valid of them).
template <int VD>
struct VRaw {
    uint32_t w[(VD + 1) / 2];
};

template <int VD>
__device__ __forceinline__ VRaw<VD> load_vraw(const uint16_t* p, bool vec, int valid) {
    VRaw<VD> r;
    if (vec && valid == VD) {
        if constexpr (VD == 1) {
            r.w[0] = p[0];
        } else if constexpr (VD == 2) {
            r.w[0] = *reinterpret_cast<const uint32_t*>(p);
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(p);
            r.w[0] = v.x;
            r.w[1] = v.y;
        }
        return r;
    }
#pragma unroll
    for (int i = 0; i < (VD + 1) / 2; ++i) r.w[i] = 0;
#pragma unroll
    for (int v = 0; v < VD; ++v)
        if (v < valid) r.w[v >> 1] |= static_cast<uint32_t>(p[v]) << (16 * (v & 1));
    return r;
}

template <int VD>
__device__ __forceinline__ void unpack_vraw(const VRaw<VD>& r, bool bf16, float* out) {
#pragma unroll
    for (int v = 0; v < VD; ++v) out[v] = rd16(static_cast<uint16_t>(r.w[v >> 1] >> (16 * (v & 1))), bf16);
}

// LDS of the split kernel, in floats: q (rows of hd + pad, padded when
// head slices read several rows at once) shares its space with `slots` (4,
// or 2 where four would pass 64 KB) of the waves' sums, then the [TOK][G]
// scores.
constexpr int kAttnLdsFloats = 16384;
__host__ __device__ constexpr int split_q_stride(int hd, int hs) { return hd + (hs > 1 ? 16 : 0); }
__host__ __device__ constexpr int split_sum_floats(int hd, int group, int hs, int slots) {
    return ((group * split_q_stride(hd, hs) > slots * group * hd ? group * split_q_stride(hd, hs) : slots * group * hd) +
            3) &
           ~3;
}

template <bool BF16, int G, int VD, int TOK>
__global__ __launch_bounds__(kAttnThreads) void attention_split_kernel(
    const float* __restrict__ q_rot, const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    int64_t kv_width, int hd, int group, int64_t T, float scale, int vec, int slots, float* __restrict__ part,
    float* __restrict__ ml) {
    constexpr int HS = G < 4 ? G : 4;         // head slices
    constexpr int HPL = G / HS;               // heads per lane in the score pass
    constexpr int NTG = kAttnThreads / (4 * HS);  // token groups in the score pass
    constexpr int TPL = TOK / NTG;            // tokens per lane in the score pass
    constexpr int NV = TOK / kAttnWaves;      // value-pass tokens per wave
    constexpr int NP = 2 * VD;                // 16-byte K pieces per quarter: hd / 32 <= 2 * VD
    static_assert(TPL >= 1 && TPL * NTG == TOK, "whole tokens per lane");
    static_assert(TPL * NP <= 16, "K pieces held in registers");
    extern __shared__ float4 sm4[];
    const int qs = split_q_stride(hd, HS);
    float* q_s = reinterpret_cast<float*>(sm4);               // [group][qs], dead after the scores
    float* buf = q_s;                                         // [slots][group][hd]: the waves' sums
    float* p_t = q_s + split_sum_floats(hd, group, HS, slots);  // [TOK][G]: scores, then weights
    const int kvh = blockIdx.x, sp = blockIdx.y, nsplit = gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t t0 = static_cast<int64_t>(sp) * TOK;
    const int n = static_cast<int>(min(static_cast<int64_t>(TOK), T - t0));

    // Every global load is issued before the first wait: this thread's K
    // pieces, its wave's V values, then the query heads into LDS.
    // score-pass lane: tokens tg, tg + NTG, ..., head slice hs, quarter qd
    const int tg = tid / (4 * HS), hs = (tid >> 2) % HS, qd = tid & 3;
    const uint16_t* kbase = k_cache + t0 * kv_width + static_cast<int64_t>(kvh) * hd;
    uint4 kraw[TPL][NP];
    if (vec) {
#pragma unroll
        for (int j = 0; j < TPL; ++j) {
            const uint16_t* kr = kbase + min(tg + NTG * j, n - 1) * kv_width;
#pragma unroll
            for (int it = 0; it < NP; ++it) {
                const int pc = qd + 4 * it;
                kraw[j][it] = 8 * pc < hd ? *reinterpret_cast<const uint4*>(kr + 8 * pc) : make_uint4(0, 0, 0, 0);
            }
        }
    }
    const int d0 = lane * VD;
    const int valid = max(0, min(VD, hd - d0));
    VRaw<VD> vraw[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int i = min(wave + u * kAttnWaves, n - 1);
        vraw[u] = load_vraw<VD>(v_cache + (t0 + i) * kv_width + static_cast<int64_t>(kvh) * hd + d0, vec != 0, valid);
    }
    {
        // the query heads: float4 pieces, all loaded before the first is stored
        const float* qsrc = q_rot + static_cast<int64_t>(kvh) * group * hd;
        if (vec) {  // hd % 8 == 0: rows of hd / 4 float4, 16-byte aligned at every kv head
            constexpr int QV = (kMaxGroup * kMaxHeadDim / 4 + kAttnThreads - 1) / kAttnThreads;
            const int hq = hd >> 2, nq = group * hq;
            float4 qv[QV];  // loaded unconditionally (clamped index), so it stays in registers
#pragma unroll
            for (int r = 0; r < QV; ++r) qv[r] = reinterpret_cast<const float4*>(qsrc)[min(tid + r * kAttnThreads, nq - 1)];
#pragma unroll
            for (int r = 0; r < QV; ++r) {
                const int i = tid + r * kAttnThreads;
                if (i < nq) {
                    const int row = i / hq;
                    reinterpret_cast<float4*>(q_s)[row * (qs >> 2) + i - row * hq] = qv[r];
                }
            }
        } else {
            for (int i = tid; i < group * hd; i += kAttnThreads) {
                const int row = i / hd;
                q_s[row * qs + i - row * hd] = qsrc[i];
            }
        }
    }
    __syncthreads();

    // Scores.  Quarter qd takes the 16-byte pieces qd, qd + 4, ... of the
    // head (8 values each), or with vec unset (head dimensions not a
    // multiple of 8) the single values qd, qd + 4, ...; head slice hs takes
    // heads hs, hs + HS, ...  Heads past `group` repeat the last one and are
    // dropped: no branch between the LDS reads, so they issue back to back.
    {
        float acc[TPL][HPL];
#pragma unroll
        for (int j = 0; j < TPL; ++j)
#pragma unroll
            for (int h = 0; h < HPL; ++h) acc[j][h] = 0.0f;
        int qrow[HPL];
#pragma unroll
        for (int h = 0; h < HPL; ++h) qrow[h] = min(hs + HS * h, group - 1) * qs;
        if (vec) {
            const float4* q4 = reinterpret_cast<const float4*>(q_s);  // qs % 4 == 0: rows stay 16-byte aligned
#pragma unroll
            for (int it = 0; it < NP; ++it) {
                const int pc = qd + 4 * it;
                if (8 * pc < hd) {
                    float4 qa[HPL], qb[HPL];
#pragma unroll
                    for (int h = 0; h < HPL; ++h) {
                        qa[h] = q4[(qrow[h] + 8 * pc) >> 2];
                        qb[h] = q4[((qrow[h] + 8 * pc) >> 2) + 1];
                    }
#pragma unroll
                    for (int j = 0; j < TPL; ++j) {
                        const uint32_t wv[4] = {kraw[j][it].x, kraw[j][it].y, kraw[j][it].z, kraw[j][it].w};
                        float kf[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            kf[e] = rd16(static_cast<uint16_t>(wv[e >> 1] >> (16 * (e & 1))), BF16);
#pragma unroll
                        for (int h = 0; h < HPL; ++h) {
                            const float qv[8] = {qa[h].x, qa[h].y, qa[h].z, qa[h].w,
                                                 qb[h].x, qb[h].y, qb[h].z, qb[h].w};
#pragma unroll
                            for (int e = 0; e < 8; ++e) acc[j][h] = fmaf(qv[e], kf[e], acc[j][h]);
                        }
                    }
                }
            }
        } else {
            for (int d = qd; d < hd; d += 4) {
                float qv[HPL];
#pragma unroll
                for (int h = 0; h < HPL; ++h) qv[h] = q_s[qrow[h] + d];
#pragma unroll
                for (int j = 0; j < TPL; ++j) {
                    const float kv = rd16(kbase[min(tg + NTG * j, n - 1) * kv_width + d], BF16);
#pragma unroll
                    for (int h = 0; h < HPL; ++h) acc[j][h] = fmaf(qv[h], kv, acc[j][h]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < TPL; ++j)
#pragma unroll
            for (int h = 0; h < HPL; ++h) {
                acc[j][h] += dpp_f32<0xB1>(acc[j][h]);  // + the xor-1 lane's quarter
                acc[j][h] += dpp_f32<0x4E>(acc[j][h]);  // + the xor-2 lanes' pair
            }
        if (qd == 0) {
#pragma unroll
            for (int j = 0; j < TPL; ++j) {
                const int t = tg + NTG * j;
#pragma unroll
                for (int h = 0; h < HPL; ++h) p_t[t * G + hs + HS * h] = t < n ? acc[j][h] * scale : -INFINITY;
            }
        }
    }
    __syncthreads();

    // Softmax: lane tt of a TOK-lane segment holds token tt of head h.
    for (int h = tid / TOK; h < group; h += kAttnThreads / TOK) {
        const int tt = tid % TOK;
        const float sc = tt < n ? p_t[tt * G + h] : -INFINITY;
        const float m = seg_max<TOK>(sc, lane);
        const float e = tt < n ? expf(sc - m) : 0.0f;
        const float l = seg_sum<TOK>(e, lane);
        p_t[tt * G + h] = e;
        if (tt == 0) {
            const int64_t slot = (static_cast<int64_t>(kvh) * nsplit + sp) * group + h;
            ml[slot * 2] = m;
            ml[slot * 2 + 1] = l;
        }
    }
    __syncthreads();

    // Values: this wave's tokens wave, wave + 4, ... (already loaded); the
    // weights of all G heads of a token are one contiguous LDS read.
    float acc[G][VD];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int v = 0; v < VD; ++v) acc[h][v] = 0.0f;
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int i = wave + u * kAttnWaves;
        if (i >= n) break;
        float vv[VD];
        unpack_vraw<VD>(vraw[u], BF16, vv);
        float pw[G];
        if constexpr (G % 4 == 0) {
#pragma unroll
            for (int h4 = 0; h4 < G / 4; ++h4) {
                const float4 w4 = reinterpret_cast<const float4*>(p_t + i * G)[h4];
                pw[4 * h4] = w4.x;
                pw[4 * h4 + 1] = w4.y;
                pw[4 * h4 + 2] = w4.z;
                pw[4 * h4 + 3] = w4.w;
            }
        } else {
#pragma unroll
            for (int h = 0; h < G; ++h) pw[h] = p_t[i * G + h];
        }
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int v = 0; v < VD; ++v) acc[h][v] = fmaf(pw[h], vv[v], acc[h][v]);
    }
    // The waves' sums go to LDS (over q, read by no wave any more).  With
    // four slots, one barrier, then each thread adds ((w0 + w2) + (w1 + w3))
    // for outputs tid, tid + 256, ..., stored 256 lanes wide.  With two,
    // waves 2 and 3 hand over first and waves 0 and 1 leave w0 + w2 and
    // w1 + w3 in their slots: the same sums, one barrier more.
    const int gh = group * hd;
    float* dst = part + (static_cast<int64_t>(kvh) * nsplit + sp) * gh;
    if (slots == 4) {
        if (valid > 0) {
#pragma unroll
            for (int h = 0; h < G; ++h)
                if (h < group)
#pragma unroll
                    for (int v = 0; v < VD; ++v)
                        if (v < valid) buf[wave * gh + h * hd + d0 + v] = acc[h][v];
        }
        __syncthreads();
        for (int i = tid; i < gh; i += kAttnThreads)
            dst[i] = (buf[i] + buf[2 * gh + i]) + (buf[gh + i] + buf[3 * gh + i]);
        return;
    }
    const int slot = wave & 1;
    if (wave >= 2 && valid > 0) {
#pragma unroll
        for (int h = 0; h < G; ++h)
            if (h < group)
#pragma unroll
                for (int v = 0; v < VD; ++v)
                    if (v < valid) buf[slot * gh + h * hd + d0 + v] = acc[h][v];
    }
    __syncthreads();
    if (wave < 2 && valid > 0) {
#pragma unroll
        for (int h = 0; h < G; ++h)
            if (h < group)
#pragma unroll
                for (int v = 0; v < VD; ++v)
                    if (v < valid) {
                        float* b = buf + slot * gh + h * hd + d0 + v;
                        *b = acc[h][v] + *b;
                    }
    }
    __syncthreads();
    for (int i = tid; i < gh; i += kAttnThreads) dst[i] = buf[i] + buf[gh + i];
}

// The launchers return false for a shape no kernel instance covers.
template <bool BF16, int G, int TOK>
bool launch_split_t(int vd, dim3 grid, size_t lds, hipStream_t st, const float* q_rot, const uint16_t* kc,
                    const uint16_t* vc, int64_t kvw, int hd, int group, int64_t T, float scale, int vec, int slots,
                    float* part, float* ml) {
    if (vd <= 1) {
        hipLaunchKernelGGL((attention_split_kernel<BF16, G, 1, TOK>), grid, dim3(kAttnThreads), lds, st, q_rot, kc, vc,
                           kvw, hd, group, T, scale, vec, slots, part, ml);
        return true;
    }
    if (vd == 2) {
        hipLaunchKernelGGL((attention_split_kernel<BF16, G, 2, TOK>), grid, dim3(kAttnThreads), lds, st, q_rot, kc, vc,
                           kvw, hd, group, T, scale, vec, slots, part, ml);
        return true;
    }
    if constexpr (8 * (TOK * (G < 4 ? G : 4) / 64) <= 16) {  // K pieces per lane: 2 * VD per token
        hipLaunchKernelGGL((attention_split_kernel<BF16, G, 4, TOK>), grid, dim3(kAttnThreads), lds, st, q_rot, kc, vc,
                           kvw, hd, group, T, scale, vec, slots, part, ml);
        return true;
    }
    return false;
}

template <bool BF16, int G>
bool launch_split_g(int tok, int vd, dim3 grid, size_t lds, hipStream_t st, const float* q_rot, const uint16_t* kc,
                    const uint16_t* vc, int64_t kvw, int hd, int group, int64_t T, float scale, int vec, int slots,
                    float* part, float* ml) {
    if constexpr (G >= 4) {
        if (tok == 16)
            return launch_split_t<BF16, G, 16>(vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec, slots,
                                               part, ml);
    }
    if constexpr (G >= 2) {
        if (tok == 32)
            return launch_split_t<BF16, G, 32>(vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec, slots,
                                               part, ml);
    }
    if (tok != 64) return false;
    return launch_split_t<BF16, G, 64>(vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec, slots, part,
                                       ml);
}

// Heads per kv head rounded up to the kernels' G.
int split_g(int group) { return group <= 1 ? 1 : (group <= 2 ? 2 : (group <= 4 ? 4 : (group <= 8 ? 8 : kMaxGroup))); }

int split_hs(int g) { return g < 4 ? g : 4; }
int split_vd(int hd) { return hd <= 64 ? 1 : (hd <= 128 ? 2 : 4); }

// Tokens per split: 64 (32 where four tokens per lane of 256-dimension heads
// would not fit the registers), halved while the launch has fewer than
// kAttnTargetGroups workgroups, down to 16 and to no fewer than the score
// pass's token groups (64 / min(G, 4)).  The work per workgroup is a chain
// of short dependent steps, so several workgroups per CU hide each other's
// latencies; the merge's cost grows only slowly with the split count.
int split_tokens(int64_t nkv, int64_t T, int g, int hd) {
    const int hs = split_hs(g);
    int tok = split_vd(hd) == 4 && hs == 4 ? kMaxSplitTokens / 2 : kMaxSplitTokens;
    while (tok > kMinSplitTokens && tok / 2 >= kMaxSplitTokens / hs && nkv * ((T + tok - 1) / tok) < kAttnTargetGroups)
        tok /= 2;
    return tok;
}

// Slots for the waves' sums: four unless that passes kAttnLdsFloats.
int split_slots(int hd, int group, int tok) {
    return split_sum_floats(hd, group, split_hs(split_g(group)), 4) + split_g(group) * tok <= kAttnLdsFloats ? 4 : 2;
}

size_t split_lds_bytes(int hd, int group, int tok, int slots) {
    return static_cast<size_t>(split_sum_floats(hd, group, split_hs(split_g(group)), slots) + split_g(group) * tok) *
           sizeof(float);
}

template <bool BF16>
bool launch_split(int tok, dim3 grid, size_t lds, hipStream_t st, const float* q_rot, const uint16_t* kc,
                  const uint16_t* vc, int64_t kvw, int hd, int group, int64_t T, float scale, int vec, int slots,
                  float* part, float* ml) {
    const int vd = split_vd(hd);
    switch (split_g(group)) {
        case 1:
            return launch_split_g<BF16, 1>(tok, vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec, slots,
                                           part, ml);
        case 2:
            return launch_split_g<BF16, 2>(tok, vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec, slots,
                                           part, ml);
        case 4:
            return launch_split_g<BF16, 4>(tok, vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec, slots,
                                           part, ml);
        case 8:
            return launch_split_g<BF16, 8>(tok, vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec, slots,
                                           part, ml);
        default:
            return launch_split_g<BF16, kMaxGroup>(tok, vd, grid, lds, st, q_rot, kc, vc, kvw, hd, group, T, scale, vec,
                                                   slots, part, ml);
    }
}

// context[h][d] = sum_s exp(m_s - M) acc_s[d] / sum_s exp(m_s - M) l_s.
// Workgroup (head, 64-dimension slice); lane = dimension, wave w takes the
// splits w, w + 16, ...  A wave issues its first kMergeBatch partials (and,
// lane u, the max of its u-th split) before anything waits, then works out M
// and the denominator itself (lanes over the splits, no barrier), so the
// partials' round trip and the (m, l) one overlap.  Lane u's exp(m_s - M)
// reaches the other lanes by readlane: one exp per lane and batch.  The 16
// waves' sums meet in LDS, added in wave order.
constexpr int kMergeBatch = 20;  // splits per wave in flight: 320 per pass

__global__ __launch_bounds__(kMergeThreads) void attention_merge_kernel(const float* __restrict__ part,
                                                                       const float* __restrict__ ml,
                                                                       float* __restrict__ context, int hd, int group,
                                                                       int nsplit) {
    constexpr int W = kMergeThreads / 64;
    constexpr int KM = 4;  // (m, l) pairs per lane kept in registers
    __shared__ float sums[W][64];
    const int head = blockIdx.x;
    const int kvh = head / group, hl = head - kvh * group;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int d = blockIdx.y * 64 + lane;
    const int dc = min(d, hd - 1);  // lanes past the head's end read a valid column and store nothing
    const int64_t base = static_cast<int64_t>(kvh) * nsplit * group + hl;  // slot of split s: base + s * group

    float pv[kMergeBatch], mlane;
    auto load_batch = [&](int s0) {
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            const int s = min(s0 + W * u, nsplit - 1);
            pv[u] = part[(base + static_cast<int64_t>(s) * group) * hd + dc];
        }
        mlane = ml[(base + static_cast<int64_t>(min(s0 + W * lane, nsplit - 1)) * group) * 2];
    };
    load_batch(wave);

    float ms[KM], ls[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        const int s = min(lane + 64 * k, nsplit - 1);
        const int64_t slot = base + static_cast<int64_t>(s) * group;
        ms[k] = ml[slot * 2];
        ls[k] = ml[slot * 2 + 1];
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (lane + 64 * k < nsplit) m = fmaxf(m, ms[k]);
    for (int s = lane + 64 * KM; s < nsplit; s += 64) m = fmaxf(m, ml[(base + static_cast<int64_t>(s) * group) * 2]);
    m = seg_max<64>(m, lane);
    float den = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (lane + 64 * k < nsplit) den += expf(ms[k] - m) * ls[k];
    for (int s = lane + 64 * KM; s < nsplit; s += 64) {
        const int64_t slot = base + static_cast<int64_t>(s) * group;
        den += expf(ml[slot * 2] - m) * ml[slot * 2 + 1];
    }
    den = seg_sum<64>(den, lane);

    float acc = 0.0f;
    for (int s0 = wave;; s0 += W * kMergeBatch) {
        const float fl = expf(mlane - m);
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u)
            if (s0 + W * u < nsplit)
                acc = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(fl), u)), pv[u], acc);
        if (s0 + W * kMergeBatch >= nsplit) break;
        load_batch(s0 + W * kMergeBatch);
    }
    sums[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && d < hd) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) t += sums[w][lane];
        context[static_cast<int64_t>(head) * hd + d] = t / den;
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
    const int tok = split_tokens(a.nkv, T, split_g(static_cast<int>(group)), static_cast<int>(hd));
    const int64_t nsplit = (T + tok - 1) / tok;
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

    const int slots = split_slots(static_cast<int>(hd), static_cast<int>(group), tok);
    const size_t lds = split_lds_bytes(static_cast<int>(hd), static_cast<int>(group), tok, slots);
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    // 16-byte K pieces need head dimensions in multiples of 8 and rows that
    // keep them aligned; the value pass's wider loads then also stay aligned
    const int vec = hd % 8 == 0 && kvw % 8 == 0 && plm::aligned16(s->k_rows(layer)) &&
                    plm::aligned16(s->v_rows(layer));
    if (!launch_split<BF16>(tok, dim3(static_cast<unsigned>(a.nkv), static_cast<unsigned>(nsplit)), lds, stream,
                            q_rot, s->k_rows(layer), s->v_rows(layer), kvw, static_cast<int>(hd),
                            static_cast<int>(group), T, scale, vec, slots, part, ml))
        return plm::fail(106, "no attention kernel for %d-token splits of head_dim %lld", tok,
                         static_cast<long long>(hd));
    if ((code = plm::check_launch("attention split")) != 0) return code;
    hipLaunchKernelGGL(attention_merge_kernel, dim3(static_cast<unsigned>(a.nh), static_cast<unsigned>((hd + 63) / 64)),
                       dim3(kMergeThreads), 0, stream,
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
