// DeepSeek session object, MoE layer entry points and routers
// (src/pcketlm/native/ds_forward.cpp:89-335, 337-367, 784-955) plus the
// DeepSeek-V3 sigmoid / grouped router of the torch runtime
// (src/pcketlm/core/runtime/fp8_source.py:1527-1547, 5125-5140) on the device.
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "common.h"
#include "route.h"

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

// DeepSeek-V3 routing, one token row per one-wave workgroup (route.h).
template <int J>
__global__ __launch_bounds__(64) void ds_route_kernel(const float* __restrict__ logits, const float* __restrict__ bias,
                                                      int experts, int top_k, int n_groups, int topk_groups,
                                                      int scoring, float route_scale, int64_t* __restrict__ out_idx,
                                                      float* __restrict__ out_w) {
    extern __shared__ float4 sh4[];  // 16-byte aligned
    float* choice = reinterpret_cast<float*>(sh4);  // [experts]
    float* score = choice + ((experts + 3) & ~3);   // [experts]
    __shared__ RouteWave rw;
    const int64_t row = blockIdx.x;
    plm_route_wave<J>(logits + row * experts, bias, experts, top_k, n_groups, topk_groups, scoring, route_scale, score,
                      choice, rw, out_idx + row * top_k, out_w + row * top_k);
}

}  // namespace

// Counters of one fused attention block call (ds_forward.cpp:775-779), for
// ds_attention_block_forward_f32 (mla.hip).  Returns 1 on a null handle.
int plm_ds_session_note_fused_attention(void* handle) {
    Session* s = static_cast<Session*>(handle);
    if (s == nullptr) return 1;
    s->monolithic_calls += 1;
    s->attention_invocations += 1;
    s->fused_attention_invocations += 1;
    return 0;
}


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

// ds_router_topk_u16 without the status read-back: the kernel's status (0,
// or 3 / 4 for a degenerate softmax sum, as the reference returns) goes to
// *status in device memory and the call returns at once.  No counterpart in
// the reference; for callers that must not wait on the stream.
PLM_EXPORT int ds_router_topk_u16_nosync(const uint16_t* hidden_u16, const uint16_t* router_weights_u16,
                                         int64_t hidden_dim, int64_t num_experts, int64_t k, int64_t dtype_code,
                                         int64_t* output_expert_ids, float* output_weights, int* status) {
    if (!hidden_u16 || !router_weights_u16 || !output_expert_ids || !output_weights || !status)
        return plm::fail(1, "null pointer");
    if (hidden_dim <= 0 || num_experts <= 0 || k <= 0 || k > num_experts) return plm::fail(2, "bad dimensions");
    hipStream_t st = plm::current_stream();
    float* ws = static_cast<float*>(plm::workspace(static_cast<size_t>(num_experts) * sizeof(float)));
    if (ws == nullptr) return plm::fail(2, "workspace");
    hipLaunchKernelGGL(softmax_router_kernel, dim3(1), dim3(256), 0, st, hidden_u16, router_weights_u16, hidden_dim,
                       num_experts, k, dtype_code, ws, output_expert_ids, output_weights, status);
    return plm::check_launch("softmax router kernel");
}

PLM_EXPORT int ds_route_topk_f32(const float* logits, const float* bias, int64_t batch, int64_t num_experts,
                                 int64_t top_k, int64_t n_groups, int64_t topk_groups, int scoring, float route_scale,
                                 int64_t* out_indices, float* out_weights) {
    if (!logits || !out_indices || !out_weights) return plm::fail(1, "null pointer");
    if (batch <= 0 || num_experts <= 0 || top_k <= 0 || top_k > num_experts || n_groups <= 0 || n_groups > 64 ||
        num_experts % n_groups != 0 || num_experts > 4096 || (scoring != 0 && scoring != 1))
        return plm::fail(2, "bad dimensions");
    const size_t shmem = static_cast<size_t>(2 * ((num_experts + 3) & ~int64_t(3))) * sizeof(float);
    const int j = plm_route_j(static_cast<int>(num_experts));
    auto kern = j == 4 ? ds_route_kernel<4> : (j == 16 ? ds_route_kernel<16> : ds_route_kernel<64>);
    hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(batch)), dim3(64), shmem, plm::current_stream(), logits, bias,
                       static_cast<int>(num_experts), static_cast<int>(top_k), static_cast<int>(n_groups),
                       static_cast<int>(topk_groups), scoring, route_scale, out_indices, out_weights);
    return plm::check_launch("ds route kernel");
}
