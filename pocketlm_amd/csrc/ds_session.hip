// DeepSeek session object, MoE layer entry points and routers
// (src/pcketlm/native/ds_forward.cpp:89-335, 337-367, 784-955) plus the
// DeepSeek-V3 sigmoid / grouped router of the torch runtime
// (src/pcketlm/core/runtime/fp8_source.py:1527-1547, 5125-5140) on the device.
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"

int plm_weighted_moe_fp8(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp,
                         const uint64_t* dp, const uint64_t* dsp, const float* hidden, const float* route,
                         float* out, int64_t experts, int64_t batch, int64_t inter, int64_t hid, int64_t gsc,
                         int64_t dsc);

namespace {

struct Registration {
    int64_t layer_idx, layer_kind, weight_role;
    const void* fp8_ptr;
    int64_t fp8_nbytes;
    const void* scale_ptr;
    int64_t scale_nbytes;
};

struct Session {
    int64_t num_layers = 0, hidden_dim = 0, num_experts = 0, top_k = 0;
    void* pack_callback = nullptr;
    void* kv_session = nullptr;
    int64_t monolithic_calls = 0;
    int64_t callback_invocations = 0;
    int64_t expert_invocations = 0;
    int64_t attention_invocations = 0;
    int64_t fused_attention_invocations = 0;
    int64_t layers_executed = 0;
    std::vector<Registration> registrations;
};

// out[i] = sum_e route[e] * outputs[e][i], products and sums rounded
// separately and experts in order (ds_forward.cpp:357-363).
__global__ void moe_combine_kernel(const float* __restrict__ outputs, const float* __restrict__ route, int64_t selected,
                                   int64_t width, float* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= width) return;
    float acc = 0.0f;
    for (int64_t e = 0; e < selected; ++e) acc = __fadd_rn(acc, __fmul_rn(route[e], outputs[e * width + i]));
    out[i] = acc;
}

__device__ __forceinline__ float u16f(uint16_t v, int64_t bf16) {
    if (bf16 == 1) return __uint_as_float(static_cast<uint32_t>(v) << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// Softmax top-k router, one workgroup (ds_forward.cpp:899-953): each thread
// scores whole experts sequentially so the fp32 sums follow the reference
// order; the normalisations are in double as in the reference.
__global__ __launch_bounds__(256) void softmax_router_kernel(const uint16_t* __restrict__ hidden,
                                                             const uint16_t* __restrict__ router, int64_t hid,
                                                             int64_t experts, int64_t k, int64_t bf16, float* scores,
                                                             int64_t* ids, float* weights, int* status) {
    for (int64_t e = threadIdx.x; e < experts; e += blockDim.x) {
        const uint16_t* row = router + e * hid;
        float acc = 0.0f;
        for (int64_t c = 0; c < hid; ++c) acc = __fadd_rn(acc, __fmul_rn(u16f(hidden[c], bf16), u16f(row[c], bf16)));
        scores[e] = acc;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    float mx = scores[0];
    for (int64_t e = 1; e < experts; ++e) mx = scores[e] > mx ? scores[e] : mx;
    double denom = 0.0;
    for (int64_t e = 0; e < experts; ++e) {
        scores[e] = expf(scores[e] - mx);
        denom += static_cast<double>(scores[e]);
    }
    if (!(denom > 0.0)) {
        *status = 3;
        return;
    }
    for (int64_t e = 0; e < experts; ++e) scores[e] = static_cast<float>(static_cast<double>(scores[e]) / denom);
    double sel = 0.0;
    for (int64_t i = 0; i < k; ++i) {
        int64_t best = -1;
        for (int64_t e = 0; e < experts; ++e) {
            bool taken = false;
            for (int64_t j = 0; j < i; ++j) taken = taken || ids[j] == e;
            if (taken) continue;
            if (best < 0 || scores[e] > scores[best]) best = e;
        }
        ids[i] = best;
        sel += static_cast<double>(scores[best]);
    }
    if (!(sel > 0.0)) {
        *status = 4;
        return;
    }
    for (int64_t i = 0; i < k; ++i) weights[i] = static_cast<float>(static_cast<double>(scores[ids[i]]) / sel);
    *status = 0;
}

__device__ __forceinline__ float bf16_round(float v) {
    // float -> bfloat16 as torch computes it here: round to nearest even,
    // every NaN -> 0xFFFF.
    const uint32_t b = __float_as_uint(v);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return __uint_as_float(0xFFFF0000u);
    return __uint_as_float(((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16) << 16);
}

// DeepSeek-V3 routing of one token row per workgroup.  Ties between exactly
// equal scores select the lower expert / group index.
__global__ __launch_bounds__(256) void ds_route_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
                                                       int64_t experts, int64_t top_k, int64_t n_groups,
                                                       int64_t topk_groups, int scoring, float route_scale,
                                                       int64_t* __restrict__ out_idx, float* __restrict__ out_w) {
    extern __shared__ float4 sh4[];  // 16-byte aligned: choice is read four values at a time
    float* score = reinterpret_cast<float*>(sh4);  // [experts]
    float* choice = score + experts;                // [experts]
    const float* lrow = logits + static_cast<int64_t>(blockIdx.x) * experts;
    if (scoring == 1) {
        // softmax in fp32
        if (threadIdx.x == 0) {
            float mx = lrow[0];
            for (int64_t e = 1; e < experts; ++e) mx = lrow[e] > mx ? lrow[e] : mx;
            float den = 0.0f;
            for (int64_t e = 0; e < experts; ++e) {
                score[e] = expf(lrow[e] - mx);
                den += score[e];
            }
            for (int64_t e = 0; e < experts; ++e) score[e] = score[e] / den;
        }
        __syncthreads();
    } else {
        for (int64_t e = threadIdx.x; e < experts; e += blockDim.x) score[e] = 1.0f / (1.0f + expf(-lrow[e]));
        __syncthreads();
    }
    for (int64_t e = threadIdx.x; e < experts; e += blockDim.x) choice[e] = bias ? score[e] + bias[e] : score[e];
    __shared__ float gscore[64];
    __shared__ int keep[64];
    __shared__ uint32_t taken[128];  // one bit per expert (at most 4096)
    __shared__ int red_first[4], red_e[4];
    __shared__ float red_v[4];
    for (int t = threadIdx.x; t < 128; t += blockDim.x) taken[t] = 0u;
    __syncthreads();
    const float ninf = -__builtin_inff();
    if (n_groups > 1) {
        // group scores, one thread per group: max, or the sum of the two
        // largest when a bias is present (the same scan as a sort's top 2)
        const int64_t gsz = experts / n_groups;
        if (threadIdx.x < n_groups) {
            const int64_t g = threadIdx.x;
            float b1 = ninf, b2 = ninf;
            for (int64_t j = 0; j < gsz; ++j) {
                const float v = choice[g * gsz + j];
                if (v > b1) {
                    b2 = b1;
                    b1 = v;
                } else if (v > b2) {
                    b2 = v;
                }
            }
            gscore[g] = bias ? b1 + b2 : b1;
            keep[g] = 0;
        }
        __syncthreads();
        const int64_t kg = topk_groups < 1 ? 1 : (topk_groups > n_groups ? n_groups : topk_groups);
        bool gnan = false;
        for (int64_t g = 0; g < n_groups; ++g) gnan = gnan || gscore[g] != gscore[g];
        if (!gnan) {
            // without NaNs the rounds keep the groups of rank < kg (a larger
            // score, or an equal one with a lower index, ranks first)
            if (threadIdx.x < n_groups) {
                const int64_t g = threadIdx.x;
                int64_t r = 0;
                for (int64_t h = 0; h < n_groups; ++h) r += gscore[h] > gscore[g] || (gscore[h] == gscore[g] && h < g);
                keep[g] = r < kg;
            }
        } else if (threadIdx.x == 0) {
            for (int64_t i = 0; i < kg; ++i) {
                int64_t best = -1;
                for (int64_t g = 0; g < n_groups; ++g)
                    if (!keep[g] && (best < 0 || gscore[g] > gscore[best])) best = g;
                keep[best] = 1;
            }
        }
        __syncthreads();
        for (int64_t e = threadIdx.x; e < experts; e += blockDim.x)
            if (!keep[e / gsz]) choice[e] = ninf;
        __syncthreads();
    }
    // Top-k as k rounds of a block-wide arg max over the experts not taken.
    // A scan in expert order keeps the first of equal values and never moves
    // off a NaN it starts from, nor onto one: so a round picks the first free
    // expert when its choice is NaN, else the largest non-NaN choice, the
    // lowest id among equals.
    const int64_t k = top_k < 1 ? 1 : (top_k > experts ? experts : top_k);
    int64_t* idx = out_idx + static_cast<int64_t>(blockIdx.x) * top_k;
    float* w = out_w + static_cast<int64_t>(blockIdx.x) * top_k;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    float sum = 0.0f;  // thread 0
    __shared__ int any_nan;
    __shared__ float pick_w[1024];  // the ranked picks' scores (at most 1024 experts there)
    __shared__ float pick_denom;
    if (threadIdx.x == 0) any_nan = 0;
    __syncthreads();
    for (int64_t e = threadIdx.x; e < experts; e += blockDim.x)
        if (choice[e] != choice[e]) any_nan = 1;
    __syncthreads();
    const bool ranked = !any_nan && experts <= 1024;
    if (ranked) {
        // Without NaNs the rounds pick the experts in the order of their rank
        // (how many experts beat them: a larger choice, or an equal one with
        // a lower id), so one pass finds all k.
        const int n = static_cast<int>(experts);
        for (int e = threadIdx.x; e < n; e += blockDim.x) {
            const float c = choice[e];
            int r = 0;
            int j = 0;
            if ((n & 3) == 0) {  // choice is then 16-byte aligned
                const float4* c4 = reinterpret_cast<const float4*>(choice);
#pragma unroll 4
                for (; j < n; j += 4) {
                    const float4 q = c4[j >> 2];
                    r += (q.x > c) || (q.x == c && j < e);
                    r += (q.y > c) || (q.y == c && j + 1 < e);
                    r += (q.z > c) || (q.z == c && j + 2 < e);
                    r += (q.w > c) || (q.w == c && j + 3 < e);
                }
            }
            for (; j < n; ++j) {
                const float cj = choice[j];
                r += (cj > c) || (cj == c && j < e);
            }
            if (r < k) {
                idx[r] = e;
                pick_w[r] = score[e];
            }
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int64_t i = 0; i < k; ++i) sum += pick_w[i];  // in pick order, as the rounds add
            pick_denom = sum > 1e-12f ? sum : 1e-12f;
        }
        __syncthreads();
        for (int64_t i = threadIdx.x; i < k; i += blockDim.x) {
            const float v = scoring == 0 ? pick_w[i] / pick_denom : pick_w[i];
            w[i] = bf16_round(v * route_scale);
        }
        return;
    }
    for (int64_t i = 0; i < (ranked ? 0 : k); ++i) {
        int first = 0x7FFFFFFF;
        int be = -1;
        float bv = ninf;
        for (int64_t e = threadIdx.x; e < experts; e += blockDim.x) {
            if ((taken[e >> 5] >> (e & 31)) & 1u) continue;
            if (first == 0x7FFFFFFF) first = static_cast<int>(e);
            const float v = choice[e];
            if (v == v && (be < 0 || v > bv)) {
                bv = v;
                be = static_cast<int>(e);
            }
        }
        for (int off = 32; off > 0; off >>= 1) {
            const int of = __shfl_xor(first, off);
            const float ov = __shfl_xor(bv, off);
            const int oe = __shfl_xor(be, off);
            first = of < first ? of : first;
            if (oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be))) {
                bv = ov;
                be = oe;
            }
        }
        if (lane == 0) {
            red_first[wave] = first;
            red_e[wave] = be;
            red_v[wave] = bv;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int t = 1; t < static_cast<int>(blockDim.x >> 6); ++t) {
                first = red_first[t] < first ? red_first[t] : first;
                const int oe = red_e[t];
                const float ov = red_v[t];
                if (oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be))) {
                    bv = ov;
                    be = oe;
                }
            }
            const float cf = choice[first];
            const int pick = (cf != cf || be < 0) ? first : be;
            idx[i] = pick;
            w[i] = score[pick];
            sum += score[pick];
            taken[pick >> 5] |= 1u << (pick & 31);
        }
        __syncthreads();
    }
    if (threadIdx.x != 0) return;
    const float denom = sum > 1e-12f ? sum : 1e-12f;
    for (int64_t i = 0; i < k; ++i) {
        const float v = scoring == 0 ? w[i] / denom : w[i];
        w[i] = bf16_round(v * route_scale);
    }
}

}  // namespace

PLM_EXPORT void* ds_session_create(int64_t num_layers, int64_t hidden_dim, int64_t num_experts, int64_t top_k,
                                   void* fp8_pack_callback, void* kv_session_handle) {
    if (num_layers <= 0 || hidden_dim <= 0 || num_experts < 0 || top_k < 0) return nullptr;
    Session* s = new (std::nothrow) Session();
    if (s == nullptr) return nullptr;
    s->num_layers = num_layers;
    s->hidden_dim = hidden_dim;
    s->num_experts = num_experts;
    s->top_k = top_k;
    s->pack_callback = fp8_pack_callback;
    s->kv_session = kv_session_handle;
    return s;
}

PLM_EXPORT void ds_session_destroy(void* handle) { delete static_cast<Session*>(handle); }

PLM_EXPORT int ds_session_register_layer(void* handle, int64_t layer_idx, int64_t layer_kind, int64_t weight_role,
                                         pocketlm_ds_tensor_callback fp8_cb, pocketlm_ds_tensor_callback scale_cb) {
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || layer_idx < 0 || layer_idx >= s->num_layers) return 1;
    if (fp8_cb == nullptr || scale_cb == nullptr) return 2;
    const void* fp8_ptr = nullptr;
    int64_t fp8_nbytes = 0;
    const int c1 = fp8_cb(layer_idx, layer_kind, weight_role, &fp8_ptr, &fp8_nbytes);
    s->callback_invocations += 1;
    if (c1 != 0 || fp8_ptr == nullptr || fp8_nbytes <= 0) return 10 + c1;
    const void* scale_ptr = nullptr;
    int64_t scale_nbytes = 0;
    const int c2 = scale_cb(layer_idx, layer_kind, weight_role, &scale_ptr, &scale_nbytes);
    s->callback_invocations += 1;
    if (c2 != 0 || scale_ptr == nullptr || scale_nbytes <= 0) return 20 + c2;
    s->registrations.push_back({layer_idx, layer_kind, weight_role, fp8_ptr, fp8_nbytes, scale_ptr, scale_nbytes});
    return 0;
}

#define PLM_COUNTER(name, field)                           \
    PLM_EXPORT int64_t name(void* handle) {                \
        Session* s = static_cast<Session*>(handle);        \
        return s == nullptr ? -1 : s->field;               \
    }
PLM_COUNTER(ds_monolithic_call_counter, monolithic_calls)
PLM_COUNTER(ds_callback_invocation_count, callback_invocations)
PLM_COUNTER(ds_expert_invocation_count, expert_invocations)
PLM_COUNTER(ds_attention_invocation_count, attention_invocations)
PLM_COUNTER(ds_fused_attention_invocation_count, fused_attention_invocations)
PLM_COUNTER(ds_layers_executed_count, layers_executed)
#undef PLM_COUNTER

PLM_EXPORT int64_t ds_registered_layer_count(void* handle) {
    Session* s = static_cast<Session*>(handle);
    return s == nullptr ? -1 : static_cast<int64_t>(s->registrations.size());
}

PLM_EXPORT int64_t ds_registered_fp8_nbytes(void* handle, int64_t index) {
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || index < 0 || index >= static_cast<int64_t>(s->registrations.size())) return -1;
    return s->registrations[static_cast<size_t>(index)].fp8_nbytes;
}

PLM_EXPORT int64_t ds_registered_scale_nbytes(void* handle, int64_t index) {
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || index < 0 || index >= static_cast<int64_t>(s->registrations.size())) return -1;
    return s->registrations[static_cast<size_t>(index)].scale_nbytes;
}

PLM_EXPORT int ds_moe_layer_forward_f32(void* handle, const float* expert_outputs, const float* route_weights,
                                        int64_t selected_count, int64_t batch, int64_t hidden_dim, float* hidden_out) {
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || !expert_outputs || !route_weights || !hidden_out) return plm::fail(1, "null pointer");
    if (selected_count <= 0 || batch <= 0 || hidden_dim <= 0) return plm::fail(2, "bad dimensions");
    const int64_t width = batch * hidden_dim;
    hipLaunchKernelGGL(moe_combine_kernel, dim3(static_cast<unsigned>(plm::ceil_div(width, 256))), dim3(256), 0,
                       plm::current_stream(), expert_outputs, route_weights, selected_count, width, hidden_out);
    const int code = plm::check_launch("moe combine kernel");
    if (code != 0) return code;
    s->monolithic_calls += 1;
    s->expert_invocations += selected_count;
    return 0;
}

PLM_EXPORT int ds_moe_layer_forward_fp8_f32(void* handle, const uint64_t* gp, const uint64_t* gsp, const uint64_t* up,
                                            const uint64_t* usp, const uint64_t* dp, const uint64_t* dsp,
                                            const float* hidden, const float* route_weights, int64_t selected_count,
                                            int64_t batch, int64_t intermediate_rows, int64_t hidden_dim,
                                            int64_t gate_scale_cols, int64_t down_scale_cols, float* hidden_out) {
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || !gp || !gsp || !up || !usp || !dp || !dsp || !hidden || !route_weights || !hidden_out)
        return plm::fail(1, "null pointer");
    if (selected_count <= 0 || batch <= 0 || intermediate_rows <= 0 || hidden_dim <= 0 || gate_scale_cols <= 0 ||
        down_scale_cols <= 0)
        return plm::fail(2, "bad dimensions");
    const int code = plm_weighted_moe_fp8(gp, gsp, up, usp, dp, dsp, hidden, route_weights, hidden_out, selected_count,
                                          batch, intermediate_rows, hidden_dim, gate_scale_cols, down_scale_cols);
    if (code != 0) return code <= -1000 ? code : 100 + code;
    s->monolithic_calls += 1;
    s->expert_invocations += selected_count;
    return 0;
}

namespace {

// The callback owns its buffer only for the duration of the call, so the
// copy is waited for before returning (the reference copies with memcpy).
int copy_callback_out(float* dst, const float* src, int64_t count) {
    const hipStream_t st = plm::current_stream();
    hipError_t err = hipMemcpyAsync(dst, src, static_cast<size_t>(count) * sizeof(float), hipMemcpyDefault, st);
    if (err == hipSuccess) err = hipStreamSynchronize(st);
    return err == hipSuccess ? 0 : plm::hip_fail(err, "callback output copy");
}

}  // namespace

PLM_EXPORT int ds_attention_layer_forward_f32(void* handle, int64_t layer_idx, const float* hidden_in, int64_t batch,
                                              int64_t hidden_dim, pocketlm_ds_attention_callback attention_callback,
                                              float* hidden_out) {
    plm::clear_error();
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || hidden_in == nullptr || attention_callback == nullptr || hidden_out == nullptr) return 1;
    if (layer_idx < 0 || layer_idx >= s->num_layers || batch <= 0 || hidden_dim <= 0) return 2;
    const float* cb_out = nullptr;
    int64_t cb_count = 0;
    const int code = attention_callback(layer_idx, hidden_in, batch, hidden_dim, &cb_out, &cb_count);
    s->callback_invocations += 1;
    if (code != 0 || cb_out == nullptr) return 10 + code;
    if (cb_count != batch * hidden_dim) return 20;
    const int c = copy_callback_out(hidden_out, cb_out, cb_count);
    if (c != 0) return c;
    s->monolithic_calls += 1;
    s->attention_invocations += 1;
    return 0;
}

PLM_EXPORT int ds_forward_decode_f32(void* handle, int64_t input_token_id, pocketlm_ds_decode_callback decode_callback,
                                     float* output_logits, int64_t vocab_size) {
    plm::clear_error();
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || decode_callback == nullptr || output_logits == nullptr) return 1;
    if (vocab_size <= 0) return 2;
    const float* cb_out = nullptr;
    int64_t cb_count = 0;
    const int code = decode_callback(input_token_id, &cb_out, &cb_count);
    s->callback_invocations += 1;
    if (code != 0 || cb_out == nullptr) return 10 + code;
    if (cb_count != vocab_size) return 20;
    const int c = copy_callback_out(output_logits, cb_out, cb_count);
    if (c != 0) return c;
    s->monolithic_calls += 1;
    s->layers_executed += s->num_layers;
    return 0;
}

PLM_EXPORT int ds_forward_prefill_f32(void* handle, const int64_t* input_token_ids, int64_t n_tokens,
                                      pocketlm_ds_prefill_callback prefill_callback, float* output_final_logits,
                                      int64_t vocab_size) {
    plm::clear_error();
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || input_token_ids == nullptr || prefill_callback == nullptr || output_final_logits == nullptr)
        return 1;
    if (n_tokens <= 0 || vocab_size <= 0) return 2;
    const float* cb_out = nullptr;
    int64_t cb_count = 0;
    const int code = prefill_callback(input_token_ids, n_tokens, &cb_out, &cb_count);
    s->callback_invocations += 1;
    if (code != 0 || cb_out == nullptr) return 10 + code;
    if (cb_count != vocab_size) return 20;
    const int c = copy_callback_out(output_final_logits, cb_out, cb_count);
    if (c != 0) return c;
    s->monolithic_calls += 1;
    s->layers_executed += s->num_layers * n_tokens;
    return 0;
}

PLM_EXPORT int ds_forward_verify_f32(void* handle, const int64_t* candidate_token_ids, int64_t k,
                                     pocketlm_ds_verify_callback verify_callback, float* output_logits_per_position,
                                     int64_t vocab_size) {
    plm::clear_error();
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr || candidate_token_ids == nullptr || verify_callback == nullptr ||
        output_logits_per_position == nullptr)
        return 1;
    if (k <= 0 || vocab_size <= 0) return 2;
    const float* cb_out = nullptr;
    int64_t cb_count = 0;
    const int code = verify_callback(candidate_token_ids, k, &cb_out, &cb_count);
    s->callback_invocations += 1;
    if (code != 0 || cb_out == nullptr) return 10 + code;
    if (cb_count != k * vocab_size) return 20;
    const int c = copy_callback_out(output_logits_per_position, cb_out, cb_count);
    if (c != 0) return c;
    s->monolithic_calls += 1;
    s->layers_executed += s->num_layers * k;
    return 0;
}

PLM_EXPORT int ds_router_topk_u16(const uint16_t* hidden_u16, const uint16_t* router_weights_u16, int64_t hidden_dim,
                                  int64_t num_experts, int64_t k, int64_t dtype_code, int64_t* output_expert_ids,
                                  float* output_weights) {
    if (!hidden_u16 || !router_weights_u16 || !output_expert_ids || !output_weights) return plm::fail(1, "null pointer");
    if (hidden_dim <= 0 || num_experts <= 0 || k <= 0 || k > num_experts) return plm::fail(2, "bad dimensions");
    hipStream_t st = plm::current_stream();
    float* ws = static_cast<float*>(plm::workspace(static_cast<size_t>(num_experts) * sizeof(float) + 64));
    if (ws == nullptr) return plm::fail(2, "workspace");
    int* status = reinterpret_cast<int*>(ws + num_experts);
    hipLaunchKernelGGL(softmax_router_kernel, dim3(1), dim3(256), 0, st, hidden_u16, router_weights_u16, hidden_dim,
                       num_experts, k, dtype_code, ws, output_expert_ids, output_weights, status);
    int code = plm::check_launch("softmax router kernel");
    if (code != 0) return code;
    // The reference reports 3 / 4 for degenerate softmax sums; read the flag.
    int host_status = 0;
    hipError_t err = hipMemcpyAsync(&host_status, status, sizeof(int), hipMemcpyDeviceToHost, st);
    if (err == hipSuccess) err = hipStreamSynchronize(st);
    if (err != hipSuccess) return plm::hip_fail(err, "router status read-back");
    return host_status;
}

PLM_EXPORT int ds_route_topk_f32(const float* logits, const float* bias, int64_t batch, int64_t num_experts,
                                 int64_t top_k, int64_t n_groups, int64_t topk_groups, int scoring, float route_scale,
                                 int64_t* out_indices, float* out_weights) {
    if (!logits || !out_indices || !out_weights) return plm::fail(1, "null pointer");
    if (batch <= 0 || num_experts <= 0 || top_k <= 0 || top_k > num_experts || n_groups <= 0 || n_groups > 64 ||
        num_experts % n_groups != 0 || num_experts > 4096 || (scoring != 0 && scoring != 1))
        return plm::fail(2, "bad dimensions");
    const size_t shmem = static_cast<size_t>(2 * num_experts) * sizeof(float);
    hipLaunchKernelGGL(ds_route_kernel, dim3(static_cast<unsigned>(batch)), dim3(256), shmem, plm::current_stream(),
                       logits, bias, num_experts, top_k, n_groups, topk_groups, scoring, route_scale, out_indices,
                       out_weights);
    return plm::check_launch("ds route kernel");
}
