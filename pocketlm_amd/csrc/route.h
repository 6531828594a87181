// DeepSeek-V3 routing of one token row, run by one wave: the torch code of
// run_fp8_router (src/pcketlm/core/runtime/fp8_source.py:1527-1547) with the
// group mask of _mask_deepseek_route_groups (5125-5140).  Shared by the
// router entry point (ds_route_topk_f32) and the MoE layer that routes its
// own logits, so both choose the same experts with the same weights.
//
// Lane l owns experts [l * J, l * J + J): their scores and choices live in
// its registers; group scores merge over DPP when groups are whole lanes;
// the top-k rounds are wave-wide arg-max reductions over DPP (no workgroup
// barrier anywhere); LDS holds only what crosses lanes (the scores read back
// by expert id, the choices scanned per group otherwise).
#pragma once

#include "common.h"

// Per-wave LDS beside the score / choice arrays.
struct RouteWave {
    float gscore[64];
    int keep[64];
};

__device__ __forceinline__ float plm_bf16_round(float v) {
    // float -> bfloat16 as torch computes it: round to nearest even, every NaN -> 0xFFFF.
    const uint32_t b = __float_as_uint(v);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float(0xFFFF0000u);
    return __uint_as_float(((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16) << 16);
}

// Orders LDS accesses of the lanes of one wave (LDS serves one wave's
// operations in issue order, so only the compiler must not move them).
__device__ __forceinline__ void plm_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int CTRL>
__device__ __forceinline__ uint32_t plm_dpp(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ uint32_t plm_readlane(uint32_t v, int lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

// DPP controls: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror.  After the four steps every lane holds the result over its
// 16-lane row; the four rows are combined from lanes 0, 16, 32 and 48.
template <int CTRL>
__device__ __forceinline__ uint64_t plm_max_step(uint64_t k) {
    const uint64_t o = (static_cast<uint64_t>(plm_dpp<CTRL>(static_cast<uint32_t>(k >> 32))) << 32) |
                       plm_dpp<CTRL>(static_cast<uint32_t>(k));
    return o > k ? o : k;
}

// The largest key of the wave, the same in every lane.  All 64 lanes active.
__device__ __forceinline__ uint64_t plm_wave_max_u64(uint64_t k) {
    k = plm_max_step<0xB1>(k);
    k = plm_max_step<0x4E>(k);
    k = plm_max_step<0x141>(k);
    k = plm_max_step<0x140>(k);
    uint64_t r = 0;
#pragma unroll
    for (int row = 0; row < 4; ++row) {
        const uint64_t v = (static_cast<uint64_t>(plm_readlane(static_cast<uint32_t>(k >> 32), 16 * row)) << 32) |
                           plm_readlane(static_cast<uint32_t>(k), 16 * row);
        r = v > r ? v : r;
    }
    return r;
}

template <int CTRL>
__device__ __forceinline__ uint32_t plm_max32_step(uint32_t v) {
    const uint32_t o = plm_dpp<CTRL>(v);
    return o > v ? o : v;
}

// The largest value of the wave, the same in every lane.  All 64 lanes active.
__device__ __forceinline__ uint32_t plm_wave_max_u32(uint32_t v) {
    v = plm_max32_step<0xB1>(v);
    v = plm_max32_step<0x4E>(v);
    v = plm_max32_step<0x141>(v);
    v = plm_max32_step<0x140>(v);
    uint32_t r = 0;
#pragma unroll
    for (int row = 0; row < 4; ++row) {
        const uint32_t o = plm_readlane(v, 16 * row);
        r = o > r ? o : r;
    }
    return r;
}

// Merges the two largest of this lane's block with those of the block the
// DPP control pairs it with (the multiset's two largest; no NaNs).
template <int CTRL>
__device__ __forceinline__ void plm_top2_step(float& b1, float& b2) {
    const float c1 = __uint_as_float(plm_dpp<CTRL>(__float_as_uint(b1)));
    const float c2 = __uint_as_float(plm_dpp<CTRL>(__float_as_uint(b2)));
    const float lo = b1 > c1 ? c1 : b1;
    const float hi2 = b2 > c2 ? b2 : c2;
    b1 = b1 > c1 ? b1 : c1;
    b2 = lo > hi2 ? lo : hi2;
}

template <int CTRL>
__device__ __forceinline__ uint32_t plm_min_step(uint32_t v) {
    const uint32_t o = plm_dpp<CTRL>(v);
    return o < v ? o : v;
}

// The smallest value of the wave, the same in every lane.  All 64 lanes active.
__device__ __forceinline__ uint32_t plm_wave_min_u32(uint32_t v) {
    v = plm_min_step<0xB1>(v);
    v = plm_min_step<0x4E>(v);
    v = plm_min_step<0x141>(v);
    v = plm_min_step<0x140>(v);
    uint32_t r = 0xFFFFFFFFu;
#pragma unroll
    for (int row = 0; row < 4; ++row) {
        const uint32_t o = plm_readlane(v, 16 * row);
        r = o < r ? o : r;
    }
    return r;
}

// A non-NaN float as an unsigned key with the float order (-0 and +0 equal);
// never 0, which stands for "none".
__device__ __forceinline__ uint32_t plm_order_key(float v) {
    uint32_t b = __float_as_uint(v);
    b = b == 0x80000000u ? 0u : b;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Arg-max key of expert e with value key o: a larger value first, then a lower id.
__device__ __forceinline__ uint64_t plm_pick_key(uint32_t o, int e) {
    return (static_cast<uint64_t>(o) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(e));
}

__device__ __forceinline__ int plm_pick_of(uint64_t key) {
    return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key));
}

// Experts per lane for a row of `experts` (at most 4096).
__host__ __device__ constexpr int plm_route_j(int experts) { return experts <= 256 ? 4 : (experts <= 1024 ? 16 : 64); }

// Routes the row lrow [experts] (fp32 logits), experts <= 64 * J.  score
// and choice are this wave's LDS arrays of experts floats (rounded up to a
// multiple of 4), 16-byte aligned.  Writes the top_k expert ids to
// idx[0..k) and their weights (rounded to bf16, as fp32) to w[0..k) in pick
// order when idx / w are not null (global or LDS memory).  When taken is
// not null, taken[lane] receives the bits j of the lane's experts
// lane * J + j that were picked, and wdense[e] (experts floats) their
// weights, 0 for the experts not picked.  Every lane of the wave calls it;
// other waves of the workgroup are not involved.
//
// The picks are those of k rounds that each take the first expert not yet
// taken when its choice is NaN, else the largest non-NaN choice not yet
// taken, the lowest id among equals; without NaNs that is the order of the
// choices, larger first, lower id first among equals.
template <int J>
__device__ __forceinline__ void plm_route_wave_generic(const float* __restrict__ lrow, const float* __restrict__ bias,
                                                       int experts, int top_k, int n_groups, int topk_groups,
                                                       int scoring, float route_scale, float* score, float* choice,
                                                       RouteWave& rw, int64_t* idx, float* w, uint64_t* taken_out,
                                                       float* wdense) {
    static_assert(J % 4 == 0 && J <= 64, "J experts per lane, a multiple of 4, at most 64");
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int e0 = lane * J;
    const float ninf = -__builtin_inff();
    const bool vec = (experts & 3) == 0 && (reinterpret_cast<uintptr_t>(lrow) & 15) == 0 &&
                     (bias == nullptr || (reinterpret_cast<uintptr_t>(bias) & 15) == 0);
    float sv[J];  // scores
    float cv[J];  // choices: scores + bias, then -inf outside the kept groups
    if (scoring == 1) {
        // softmax in fp32, one lane, in expert order
        if (lane == 0) {
            float mx = lrow[0];
            for (int e = 1; e < experts; ++e) mx = lrow[e] > mx ? lrow[e] : mx;
            float den = 0.0f;
            for (int e = 0; e < experts; ++e) {
                score[e] = expf(lrow[e] - mx);
                den += score[e];
            }
            for (int e = 0; e < experts; ++e) score[e] = score[e] / den;
        }
        plm_wave_sync();
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int e = e0 + j;
            sv[j] = e < experts ? score[e] : 0.0f;
        }
    } else {
#pragma unroll
        for (int q = 0; q < J / 4; ++q) {
            const int e = e0 + 4 * q;
            float x[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (vec) {
                if (e < experts) {
                    const float4 v = *reinterpret_cast<const float4*>(lrow + e);
                    x[0] = v.x;
                    x[1] = v.y;
                    x[2] = v.z;
                    x[3] = v.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) x[i] = e + i < experts ? lrow[e + i] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[4 * q + i] = 1.0f / (1.0f + expf(-x[i]));
            if (vec) {
                if (e < experts)
                    *reinterpret_cast<float4*>(score + e) = make_float4(sv[4 * q], sv[4 * q + 1], sv[4 * q + 2],
                                                                        sv[4 * q + 3]);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (e + i < experts) score[e + i] = sv[4 * q + i];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) cv[j] = sv[j];
    if (bias != nullptr) {
#pragma unroll
        for (int q = 0; q < J / 4; ++q) {
            const int e = e0 + 4 * q;
            if (vec) {
                if (e < experts) {
                    const float4 b = *reinterpret_cast<const float4*>(bias + e);
                    cv[4 * q] += b.x;
                    cv[4 * q + 1] += b.y;
                    cv[4 * q + 2] += b.z;
                    cv[4 * q + 3] += b.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (e + i < experts) cv[4 * q + i] += bias[e + i];
            }
        }
    }
    if (n_groups > 1) {
        // Group scores: the max, or the sum of the two largest when a bias
        // is present (the same values as an in-order scan that passes over
        // NaNs and counts equal values twice: the multiset's two largest).
        const int gsz = experts / n_groups;
        const int lg = gsz / J;  // lanes per group, when groups are whole lanes
        const bool lane_groups = gsz % J == 0 && (lg == 1 || lg == 2 || lg == 4 || lg == 8 || lg == 16);
        float gs = ninf;    // lane g < n_groups: group g's score
        float mine = ninf;  // lane_groups: the score of this lane's group
        if (lane_groups) {
            // each lane's two largest, then merged over the group's lanes
            float b1 = ninf, b2 = ninf;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const float v = cv[j];
                const bool gt1 = v > b1, gt2 = v > b2;
                b2 = gt1 ? b1 : (gt2 ? v : b2);
                b1 = gt1 ? v : b1;
            }
            if (lg >= 2) plm_top2_step<0xB1>(b1, b2);
            if (lg >= 4) plm_top2_step<0x4E>(b1, b2);
            if (lg >= 8) plm_top2_step<0x141>(b1, b2);
            if (lg >= 16) plm_top2_step<0x140>(b1, b2);
            mine = bias != nullptr ? b1 + b2 : b1;
            gs = __shfl(mine, (lane * lg) & 63);
        } else {
#pragma unroll
            for (int q = 0; q < J / 4; ++q) {
                const int e = e0 + 4 * q;
                if (vec) {
                    if (e < experts)
                        *reinterpret_cast<float4*>(choice + e) = make_float4(cv[4 * q], cv[4 * q + 1],
                                                                             cv[4 * q + 2], cv[4 * q + 3]);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (e + i < experts) choice[e + i] = cv[4 * q + i];
                }
            }
            plm_wave_sync();
            if (lane < n_groups) {
                float b1 = ninf, b2 = ninf;
                const float* g = choice + lane * gsz;
                for (int j = 0; j < gsz; ++j) {
                    const float v = g[j];
                    const bool gt1 = v > b1, gt2 = v > b2;
                    b2 = gt1 ? b1 : (gt2 ? v : b2);
                    b1 = gt1 ? v : b1;
                }
                gs = bias != nullptr ? b1 + b2 : b1;
                rw.gscore[lane] = gs;
            }
            plm_wave_sync();
        }
        const int kg = topk_groups < 1 ? 1 : (topk_groups > n_groups ? n_groups : topk_groups);
        const bool gnan = __ballot(lane < n_groups && gs != gs) != 0;
        uint64_t keep;
        if (!gnan) {
            // without NaNs the rounds keep the groups of rank < kg (a larger
            // score, or an equal one with a lower index, ranks first)
            int r = 0;
            if (lane_groups) {
                for (int h = 0; h < n_groups; ++h) {
                    const float o = __uint_as_float(plm_readlane(__float_as_uint(mine), h * lg));
                    r += o > gs || (o == gs && h < lane);
                }
            } else if (lane < n_groups) {
                for (int h = 0; h < n_groups; ++h) {
                    const float o = rw.gscore[h];
                    r += o > gs || (o == gs && h < lane);
                }
            }
            keep = __ballot(lane < n_groups && r < kg);
        } else {
            // kg rounds: the first group not kept, replaced by any later
            // one with a larger score (a NaN score is never replaced)
            if (lane < n_groups) rw.gscore[lane] = gs;
            plm_wave_sync();
            if (lane == 0) {
                for (int h = 0; h < n_groups; ++h) rw.keep[h] = 0;
                for (int i = 0; i < kg; ++i) {
                    int best = -1;
                    for (int g = 0; g < n_groups; ++g)
                        if (!rw.keep[g] && (best < 0 || rw.gscore[g] > rw.gscore[best])) best = g;
                    rw.keep[best] = 1;
                }
            }
            plm_wave_sync();
            keep = __ballot(lane < n_groups && rw.keep[lane]);
        }
        int g = e0 / gsz;
        int next = (g + 1) * gsz;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int e = e0 + j;
            if (e >= next) {  // gsz >= 1: at most one group boundary per expert
                ++g;
                next += gsz;
            }
            const bool kp = g < n_groups && ((keep >> g) & 1ull);
            if (!kp) cv[j] = ninf;
        }
    }
    // Top-k rounds.  key[j]: the order key of a free non-NaN choice, else 0;
    // taken: bit j set when expert e0 + j is out of range or taken.
    const int k = top_k < 1 ? 1 : (top_k > experts ? experts : top_k);
    uint64_t taken = 0;
    bool has_nan = false;
    uint32_t key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool in = e0 + j < experts;
        if (!in) taken |= 1ull << j;
        has_nan = has_nan || (in && cv[j] != cv[j]);
        key[j] = in && cv[j] == cv[j] ? plm_order_key(cv[j]) : 0u;
    }
    const uint64_t outside = taken;
    const bool any_nan = __ballot(has_nan) != 0;
    int* picks = reinterpret_cast<int*>(choice);  // the choices are in registers from here on
    plm_wave_sync();
    for (int i = 0; i < k; ++i) {
        // this lane's best (strict: the lowest id among equals)
        uint32_t bo = key[0];
        int bj = 0;
#pragma unroll
        for (int j = 1; j < J; ++j) {
            const bool better = key[j] > bo;
            bo = better ? key[j] : bo;
            bj = better ? j : bj;
        }
        // the largest over the wave; the lowest lane holding it holds the lowest id
        const uint32_t top = plm_wave_max_u32(bo);
        const uint64_t hit = __ballot(top != 0 && bo == top);
        const int owner = hit != 0 ? static_cast<int>(__builtin_ctzll(hit)) : 0;
        int pick = static_cast<int>(plm_readlane(static_cast<uint32_t>(e0 + bj), owner));
        if (any_nan) {
            int lf = INT32_MAX, ln = INT32_MAX;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                if ((taken >> j) & 1ull) continue;
                lf = lf == INT32_MAX ? e0 + j : lf;
                if (cv[j] != cv[j]) ln = ln == INT32_MAX ? e0 + j : ln;
            }
            const uint32_t first = plm_wave_min_u32(static_cast<uint32_t>(lf));
            const uint32_t first_nan = plm_wave_min_u32(static_cast<uint32_t>(ln));
            if (first == first_nan || top == 0) pick = static_cast<int>(first);
        }
        if (pick >= e0 && pick < e0 + J) {
            taken |= 1ull << (pick - e0);
#pragma unroll
            for (int j = 0; j < J; ++j) key[j] = pick == e0 + j ? 0u : key[j];
        }
        if (lane == 0) picks[i] = pick;
    }
    plm_wave_sync();
    // the picks' scores, added in pick order as the rounds add them
    float sum = 0.0f;
    int p0 = 0;
    float s0 = 0.0f;
    for (int i0 = 0; i0 < k; i0 += 64) {
        const int i = i0 + lane;
        const int p = i < k ? picks[i] : 0;
        const float s = i < k ? score[p] : 0.0f;
        if (i0 == 0) {
            p0 = p;
            s0 = s;
        }
        const int cnt = k - i0 < 64 ? k - i0 : 64;
        for (int t = 0; t < cnt; ++t) sum += __uint_as_float(plm_readlane(__float_as_uint(s), t));
    }
    const float denom = sum > 1e-12f ? sum : 1e-12f;
    if (taken_out != nullptr) {
        const uint64_t mine = taken & ~outside;
        taken_out[lane] = mine;
#pragma unroll
        for (int q = 0; q < J / 4; ++q) {
            float4 v;
            float* vp = reinterpret_cast<float*>(&v);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int j = 4 * q + i;
                const float x = scoring == 0 ? sv[j] / denom : sv[j];
                vp[i] = ((mine >> j) & 1ull) ? plm_bf16_round(x * route_scale) : 0.0f;
            }
            if (e0 + 4 * q < experts) *reinterpret_cast<float4*>(wdense + e0 + 4 * q) = v;
        }
    }
    if (idx != nullptr)
        for (int i = lane; i < k; i += 64) {
            const int p = i < 64 ? p0 : picks[i];
            const float s = i < 64 ? s0 : score[p];
            const float v = scoring == 0 ? s / denom : s;
            idx[i] = p;
            w[i] = plm_bf16_round(v * route_scale);
        }
    plm_wave_sync();
}

// The same routing for the common case, in registers and without LDS:
// 4 experts per lane (at most 256), a multiple of 4 of them, 16-byte aligned
// logits and bias, sigmoid scores, and either no groups or groups of whole
// lanes.  Returns false, having written nothing, when the row falls outside
// that case or holds a NaN choice or group score; the caller then runs the
// general version.  The arithmetic is the general version's, step for step
// (the same scores, group ranks, pick rounds, sum order and weight rounding),
// so the two agree bit for bit wherever this one applies.
__device__ __forceinline__ bool plm_route_wave4_fast(const float* __restrict__ lrow, const float* __restrict__ bias,
                                                     int experts, int top_k, int n_groups, int topk_groups,
                                                     int scoring, float route_scale, int64_t* idx, float* w,
                                                     uint64_t* taken_out, float* wdense) {
    constexpr int J = 4;
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int e0 = lane * J;
    const float ninf = -__builtin_inff();
    if (scoring != 0 || experts > 64 * J || (experts & 3) != 0 || top_k > 64 || (reinterpret_cast<uintptr_t>(lrow) & 15) != 0 ||
        (bias != nullptr && (reinterpret_cast<uintptr_t>(bias) & 15) != 0))
        return false;
    const int gsz = n_groups > 1 ? experts / n_groups : experts;
    const int lg = gsz / J;
    if (n_groups > 1 && !(gsz % J == 0 && (lg == 1 || lg == 2 || lg == 4 || lg == 8 || lg == 16))) return false;
    const bool own = e0 < experts;
    const float4 xv = *reinterpret_cast<const float4*>(lrow + (own ? e0 : 0));
    const float4 bv = bias != nullptr ? *reinterpret_cast<const float4*>(bias + (own ? e0 : 0))
                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float x[4] = {own ? xv.x : 0.0f, own ? xv.y : 0.0f, own ? xv.z : 0.0f, own ? xv.w : 0.0f};
    const float bb[4] = {bv.x, bv.y, bv.z, bv.w};
    float sv[J], cv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        sv[j] = 1.0f / (1.0f + expf(-x[j]));
        cv[j] = sv[j];
    }
    if (bias != nullptr && own) {
#pragma unroll
        for (int j = 0; j < J; ++j) cv[j] += bb[j];
    }
    bool nan = false;
#pragma unroll
    for (int j = 0; j < J; ++j) nan = nan || (own && cv[j] != cv[j]);
    if (__ballot(nan) != 0) return false;
    if (n_groups > 1) {
        float b1 = ninf, b2 = ninf;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const float v = cv[j];
            const bool gt1 = v > b1, gt2 = v > b2;
            b2 = gt1 ? b1 : (gt2 ? v : b2);
            b1 = gt1 ? v : b1;
        }
        if (lg >= 2) plm_top2_step<0xB1>(b1, b2);
        if (lg >= 4) plm_top2_step<0x4E>(b1, b2);
        if (lg >= 8) plm_top2_step<0x141>(b1, b2);
        if (lg >= 16) plm_top2_step<0x140>(b1, b2);
        const float mine = bias != nullptr ? b1 + b2 : b1;
        const float gs = __shfl(mine, (lane * lg) & 63);
        if (__ballot(lane < n_groups && gs != gs) != 0) return false;
        const int kg = topk_groups < 1 ? 1 : (topk_groups > n_groups ? n_groups : topk_groups);
        int r = 0;
        for (int h = 0; h < n_groups; ++h) {
            const float o = __uint_as_float(plm_readlane(__float_as_uint(mine), h * lg));
            r += o > gs || (o == gs && h < lane);
        }
        const uint64_t keep = __ballot(lane < n_groups && r < kg);
        const int g = lane / lg;
        if (!(g < n_groups && ((keep >> g) & 1ull))) {
#pragma unroll
            for (int j = 0; j < J; ++j) cv[j] = ninf;
        }
    }
    const int k = top_k < 1 ? 1 : (top_k > experts ? experts : top_k);
    uint32_t key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) key[j] = own ? plm_order_key(cv[j]) : 0u;
    uint64_t taken = 0;
    int my_pick = 0;
    float my_s = 0.0f, sum = 0.0f;
    for (int i = 0; i < k; ++i) {
        uint32_t bo = key[0];
        int bj = 0;
        float bs = sv[0];
#pragma unroll
        for (int j = 1; j < J; ++j) {
            const bool better = key[j] > bo;
            bo = better ? key[j] : bo;
            bj = better ? j : bj;
            bs = better ? sv[j] : bs;
        }
        const uint32_t top = plm_wave_max_u32(bo);
        const uint64_t hit = __ballot(top != 0 && bo == top);
        const int owner = hit != 0 ? static_cast<int>(__builtin_ctzll(hit)) : 0;
        const int pick = static_cast<int>(plm_readlane(static_cast<uint32_t>(e0 + bj), owner));
        const float s = __uint_as_float(plm_readlane(__float_as_uint(bs), owner));
        if (lane == owner) {
            taken |= 1ull << bj;
#pragma unroll
            for (int j = 0; j < J; ++j) key[j] = j == bj ? 0u : key[j];
        }
        my_pick = lane == i ? pick : my_pick;
        my_s = lane == i ? s : my_s;
        sum += s;
    }
    const float denom = sum > 1e-12f ? sum : 1e-12f;
    if (taken_out != nullptr) {
        taken_out[lane] = taken;
        if (own) {
            float4 v;
            float* vp = reinterpret_cast<float*>(&v);
#pragma unroll
            for (int j = 0; j < J; ++j) vp[j] = ((taken >> j) & 1ull) ? plm_bf16_round((sv[j] / denom) * route_scale) : 0.0f;
            *reinterpret_cast<float4*>(wdense + e0) = v;
        }
    }
    if (idx != nullptr && lane < k) {
        idx[lane] = my_pick;
        w[lane] = plm_bf16_round((my_s / denom) * route_scale);
    }
    plm_wave_sync();
    return true;
}

// The general version out of line: the common case stays a short stretch
// of straight-line code.
template <int J>
__device__ __noinline__ void plm_route_wave_cold(const float* __restrict__ lrow, const float* __restrict__ bias,
                                                 int experts, int top_k, int n_groups, int topk_groups, int scoring,
                                                 float route_scale, float* score, float* choice, RouteWave& rw,
                                                 int64_t* idx, float* w, uint64_t* taken_out, float* wdense) {
    plm_route_wave_generic<J>(lrow, bias, experts, top_k, n_groups, topk_groups, scoring, route_scale, score, choice,
                              rw, idx, w, taken_out, wdense);
}

// Routes one row: the register version where it applies (4 experts per
// lane), else the general one.  Arguments as plm_route_wave_generic's.
template <int J>
__device__ __forceinline__ void plm_route_wave(const float* __restrict__ lrow, const float* __restrict__ bias,
                                               int experts, int top_k, int n_groups, int topk_groups, int scoring,
                                               float route_scale, float* score, float* choice, RouteWave& rw,
                                               int64_t* idx, float* w, uint64_t* taken_out = nullptr,
                                               float* wdense = nullptr) {
    if constexpr (J == 4) {
        if (plm_route_wave4_fast(lrow, bias, experts, top_k, n_groups, topk_groups, scoring, route_scale, idx, w,
                                 taken_out, wdense))
            return;
        plm_route_wave_cold<4>(lrow, bias, experts, top_k, n_groups, topk_groups, scoring, route_scale, score, choice,
                               rw, idx, w, taken_out, wdense);
    } else {
        plm_route_wave_generic<J>(lrow, bias, experts, top_k, n_groups, topk_groups, scoring, route_scale, score,
                                  choice, rw, idx, w, taken_out, wdense);
    }
}
