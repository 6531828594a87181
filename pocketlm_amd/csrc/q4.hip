// Q4 kernels for gfx950: dequant (src/pcketlm/native/q4_dequant.cpp:171-286),
// the per-row Q4 dot and the fused one-token SwiGLU MoE (357-476).
//
// Format (src/pcketlm/core/model_import/q4_quantize.py:21-71): signed
// two's-complement nibbles flat over the tensor, element 2i in the low
// nibble of byte i, one fp16 scale per channel (row).
//
// Dot products.  A lane reads 16 packed bytes (32 values) per load.  Each
// dword d holds 8 nibbles; u = d ^ 0x88888888 turns every signed nibble q
// into the unsigned u = q + 8, so (u & 0x0F0F0F0F) and ((u >> 4) & ...) give
// the even / odd elements as bytes, which v_cvt_f32_ubyte{0..3} turn into
// floats with no per-element extract.  The +8 bias is removed once per
// 32-value span: sum(q*x) = sum(u*x) - 8*sum(x), where sum(x) over the span
// is shared by every row of the tile.  The row scale multiplies the span sum.
#include <algorithm>
#include <cstring>
#include <vector>

#include "common.h"

namespace {

constexpr int kMaxGroups = 64;
constexpr int kMaxWaves = 8;

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// fp16 -> fp32 as the reference's software converter (q4_dequant.cpp:10-40):
// exact for numbers, NaN payload kept without forcing the quiet bit.
__device__ __forceinline__ float h2f_ref(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    const _Float16 hv = __builtin_bit_cast(_Float16, h);
    return static_cast<float>(hv);
}

__device__ __forceinline__ bool nan_bits(uint32_t b) { return (b & 0x7FFFFFFFu) > 0x7F800000u; }

// Bits of the x86 product q * scale (q is a small integer, never NaN).
__device__ __forceinline__ uint32_t q_mul_bits(float q, float s) {
    if (nan_bits(f2u(s))) return f2u(s) | 0x00400000u;
    const float r = q * s;
    return r != r ? 0xFFC00000u : f2u(r);
}

__device__ __forceinline__ uint16_t f16_rne_hw(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// fp32 -> fp16 as F16C (vector path) or as the software converter (tail),
// which differ only for NaN.
__device__ __forceinline__ uint16_t f16_from_bits(uint32_t b, bool f16c) {
    if (nan_bits(b)) {
        const uint32_t sign = (b >> 16) & 0x8000u, mant = (b & 0x7FFFFFu) >> 13;
        return static_cast<uint16_t>(f16c ? (sign | 0x7E00u | mant) : (sign | 0x7C00u | mant | 1u));
    }
    return f16_rne_hw(u2f(b));
}

__device__ __forceinline__ int q4_at(const uint8_t* p, int64_t idx) {
    const int byte = p[idx >> 1];
    const int n = (idx & 1) ? (byte >> 4) : (byte & 0xF);
    return n >= 8 ? n - 16 : n;
}

// ------------------------------------------------------------------ dequant

// Fast path: channel_size % 32 == 0; one thread = 16 packed bytes = 32 values.
__global__ __launch_bounds__(256) void q4_dequant_kernel(const uint8_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         uint16_t* __restrict__ out, int64_t nvec,
                                                         uint32_t vec_per_channel) {
    const int64_t v = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (v >= nvec) return;
    const int64_t c = static_cast<uint64_t>(v) / vec_per_channel;
    const float sc = h2f_ref(scales[c]);
    const uint4 q = *reinterpret_cast<const uint4*>(packed + v * 16);
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    uint32_t h[16];
    const bool finite = (f2u(sc) & 0x7F800000u) != 0x7F800000u;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            // sign-extend nibble k / k+1 (compiles to v_bfe_i32)
            const float q0 = static_cast<float>(static_cast<int>(d[i] << (28 - 4 * k)) >> 28);
            const float q1 = static_cast<float>(static_cast<int>(d[i] << (24 - 4 * k)) >> 28);
            uint32_t lo, hi;
            if (finite) {
                lo = f16_rne_hw(q0 * sc);
                hi = f16_rne_hw(q1 * sc);
            } else {
                lo = f16_from_bits(q_mul_bits(q0, sc), true);
                hi = f16_from_bits(q_mul_bits(q1, sc), true);
            }
            h[i * 4 + k / 2] = lo | (hi << 16);
        }
    }
    uint4* o = reinterpret_cast<uint4*>(out + v * 32);
    o[0] = make_uint4(h[0], h[1], h[2], h[3]);
    o[1] = make_uint4(h[4], h[5], h[6], h[7]);
    o[2] = make_uint4(h[8], h[9], h[10], h[11]);
    o[3] = make_uint4(h[12], h[13], h[14], h[15]);
}

// Any shape: one thread per value, choosing the reference's converter per
// element (F16C inside its 16-value blocks when the channel starts on an even
// value index, the software converter otherwise).
__global__ void q4_dequant_scalar_kernel(const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                                         int64_t channels, int64_t cs) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= channels * cs) return;
    const int64_t c = idx / cs;
    const int64_t i = idx - c * cs;
    const float sc = h2f_ref(scales[c]);
    const bool vec = ((c * cs) & 1) == 0 && i < (cs / 16) * 16;
    out[idx] = f16_from_bits(q_mul_bits(static_cast<float>(q4_at(packed, idx)), sc), vec);
}

int q4_dequant_launch(const uint8_t* packed, const uint16_t* scales, uint16_t* out, int64_t channels, int64_t cs,
                      hipStream_t st) {
    const int64_t total = channels * cs;
    if (total <= 0) return 0;
    if (cs % 32 == 0 && plm::aligned16(packed) && plm::aligned16(out) && cs / 32 <= 0xFFFFFFFFll) {
        const int64_t nvec = total / 32;
        hipLaunchKernelGGL(q4_dequant_kernel, dim3(static_cast<unsigned>(plm::ceil_div(nvec, 256))), dim3(256), 0, st,
                           packed, scales, out, nvec, static_cast<uint32_t>(cs / 32));
    } else {
        hipLaunchKernelGGL(q4_dequant_scalar_kernel, dim3(static_cast<unsigned>(plm::ceil_div(total, 256))),
                           dim3(256), 0, st, packed, scales, out, channels, cs);
    }
    return plm::check_launch("q4 dequant kernel");
}

// ------------------------------------------------------------------ dot products

// sum over the 32 values of one 16-byte span of (u * x), with u = q + 8.
__device__ __forceinline__ float span_dot_u(const uint4& q, const float* x) {
    const uint32_t d[4] = {q.x ^ 0x88888888u, q.y ^ 0x88888888u, q.z ^ 0x88888888u, q.w ^ 0x88888888u};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = d[i] & 0x0F0F0F0Fu;
        const uint32_t hi = (d[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float ue = static_cast<float>((lo >> (8 * b)) & 0xFFu);
            const float uo = static_cast<float>((hi >> (8 * b)) & 0xFFu);
            p = fmaf(ue, x[i * 8 + 2 * b], p);
            p = fmaf(uo, x[i * 8 + 2 * b + 1], p);
        }
    }
    return p;
}

template <bool XF16>
__device__ __forceinline__ void load_x32(const void* xbase, int64_t col, float* x) {
    if constexpr (XF16) {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xbase) + col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 v = p[i];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[i * 8 + 2 * j] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[j] & 0xFFFFu)));
                x[i * 8 + 2 * j + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w[j] >> 16)));
            }
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(xbase) + col);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = p[i];
            x[4 * i] = v.x;
            x[4 * i + 1] = v.y;
            x[4 * i + 2] = v.z;
            x[4 * i + 3] = v.w;
        }
    }
}

__device__ __forceinline__ float sum32(const float* x) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) s += x[j];
    return s;
}

struct Q4RowsArgs {
    const uint8_t* w[2][kMaxGroups];
    const uint16_t* s[2][kMaxGroups];
    const void* x;        // fp16 or fp32 activations [K]
    float* out;           // (g, row) at g * rows + row
    int64_t rows;
    int64_t K;            // values per row (multiple of 32 on this path)
    int tiles_per_group;
    int nchunks;          // ceil(K/2 / 1024)
};

// Rows of one or more experts against one shared activation vector.  NWT=2
// with SILU computes silu(gate) * up (the gate/up phase of the MoE).
template <int TR, int NWT, bool SILU, bool XF16>
__global__ __launch_bounds__(512) void q4_rows_kernel(const Q4RowsArgs a) {
    constexpr int V = NWT * TR;
    __shared__ float red[kMaxWaves * V];
    const int nw = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int g = blockIdx.x / a.tiles_per_group;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x - g * a.tiles_per_group) * TR;
    const int64_t row_bytes = a.K >> 1;

    float acc[NWT][TR];
#pragma unroll
    for (int i = 0; i < NWT; ++i)
#pragma unroll
        for (int r = 0; r < TR; ++r) acc[i][r] = 0.0f;

    for (int c = wave; c < a.nchunks; c += nw) {
        const int64_t byte = static_cast<int64_t>(c) * plm::kChunkBytes + lane * 16;
        if (byte >= row_bytes) continue;
        uint4 q[NWT][TR];
#pragma unroll
        for (int i = 0; i < NWT; ++i)
#pragma unroll
            for (int r = 0; r < TR; ++r) {
                q[i][r] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
                if (row0 + r < a.rows)
                    q[i][r] = *reinterpret_cast<const uint4*>(a.w[i][g] + (row0 + r) * row_bytes + byte);
            }
        float x[32];
        load_x32<XF16>(a.x, byte * 2, x);
        const float xs8 = 8.0f * sum32(x);
#pragma unroll
        for (int i = 0; i < NWT; ++i)
#pragma unroll
            for (int r = 0; r < TR; ++r) acc[i][r] += span_dot_u(q[i][r], x) - xs8;
    }

#pragma unroll
    for (int i = 0; i < NWT; ++i)
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            const float t = plm_wave_sum(acc[i][r]);
            if (lane == 0) red[wave * V + i * TR + r] = t;
        }
    __syncthreads();
    if (threadIdx.x < TR) {
        const int r = threadIdx.x;
        const int64_t row = row0 + r;
        if (row < a.rows) {
            float v[NWT];
#pragma unroll
            for (int i = 0; i < NWT; ++i) {
                float s = 0.0f;
                for (int w = 0; w < nw; ++w) s += red[w * V + i * TR + r];
                v[i] = s * h2f_ref(a.s[i][g][row]);
            }
            if constexpr (SILU) {
                a.out[static_cast<int64_t>(g) * a.rows + row] = plm_silu_mul(v[0], v[1]);
            } else {
                a.out[static_cast<int64_t>(g) * a.rows + row] = v[0];
            }
        }
    }
}

struct Q4CombineArgs {
    const uint8_t* w[kMaxGroups];
    const uint16_t* s[kMaxGroups];
    const float* act;     // [ngroups][K] fp32
    const float* route;   // [ngroups]
    uint16_t* out_f16;    // [rows]
    int64_t rows;
    int64_t K;
    int ngroups;
    int cps;
};

// Down phase + routed combine of the Q4 MoE, fp16 out (software RNE).
template <int TR>
__global__ __launch_bounds__(512) void q4_combine_kernel(const Q4CombineArgs a) {
    __shared__ float red[kMaxWaves * TR];
    const int nw = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * TR;
    const int64_t row_bytes = a.K >> 1;
    float acc[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) acc[r] = 0.0f;
    const int nchunks = a.ngroups * a.cps;
    for (int c = wave; c < nchunks; c += nw) {
        const int g = c / a.cps;
        const int64_t byte = static_cast<int64_t>(c - g * a.cps) * plm::kChunkBytes + lane * 16;
        if (byte >= row_bytes) continue;
        uint4 q[TR];
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            q[r] = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
            if (row0 + r < a.rows) q[r] = *reinterpret_cast<const uint4*>(a.w[g] + (row0 + r) * row_bytes + byte);
        }
        float x[32];
        load_x32<false>(a.act + static_cast<int64_t>(g) * a.K, byte * 2, x);
        const float xs8 = 8.0f * sum32(x);
        const float rw = a.route[g];
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            const float sc = (row0 + r < a.rows) ? h2f_ref(a.s[g][row0 + r]) : 0.0f;
            acc[r] = fmaf((span_dot_u(q[r], x) - xs8) * sc, rw, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const float t = plm_wave_sum(acc[r]);
        if (lane == 0) red[wave * TR + r] = t;
    }
    __syncthreads();
    if (threadIdx.x < TR) {
        const int64_t row = row0 + threadIdx.x;
        if (row < a.rows) {
            float v = 0.0f;
            for (int w = 0; w < nw; ++w) v += red[w * TR + threadIdx.x];
            a.out_f16[row] = f16_from_bits(f2u(v), false);
        }
    }
}

// Any shape: one thread per (group, row).
template <bool XF16>
__global__ void q4_rows_scalar_kernel(const Q4RowsArgs a, int ngroups, int nwt, int silu) {
    const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (id >= ngroups * a.rows) return;
    const int g = static_cast<int>(id / a.rows);
    const int64_t row = id - static_cast<int64_t>(g) * a.rows;
    float v[2] = {0.0f, 0.0f};
    for (int i = 0; i < nwt; ++i) {
        float s = 0.0f;
        for (int64_t k = 0; k < a.K; ++k) {
            const float xv = XF16 ? static_cast<float>(__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(a.x)[k]))
                                  : static_cast<const float*>(a.x)[k];
            s = fmaf(static_cast<float>(q4_at(a.w[i][g], row * a.K + k)), xv, s);
        }
        v[i] = s * h2f_ref(a.s[i][g][row]);
    }
    a.out[id] = silu ? plm_silu_mul(v[0], v[1]) : v[0];
}

__global__ void q4_combine_scalar_kernel(const Q4CombineArgs a) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= a.rows) return;
    float acc = 0.0f;
    for (int g = 0; g < a.ngroups; ++g) {
        float s = 0.0f;
        for (int64_t k = 0; k < a.K; ++k)
            s = fmaf(static_cast<float>(q4_at(a.w[g], row * a.K + k)), a.act[static_cast<int64_t>(g) * a.K + k], s);
        acc = fmaf(s * h2f_ref(a.s[g][row]), a.route[g], acc);
    }
    a.out_f16[row] = f16_from_bits(f2u(acc), false);
}

int waves_for(int64_t nchunks) { return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(nchunks, kMaxWaves))); }

template <int TR, int NWT, bool SILU, bool XF16>
void launch_q4_rows(Q4RowsArgs a, int ngroups, hipStream_t st) {
    a.tiles_per_group = static_cast<int>(plm::ceil_div(a.rows, TR));
    a.nchunks = static_cast<int>(plm::ceil_div(a.K / 2, plm::kChunkBytes));
    const int nw = waves_for(a.nchunks);
    hipLaunchKernelGGL((q4_rows_kernel<TR, NWT, SILU, XF16>),
                       dim3(static_cast<unsigned>(static_cast<int64_t>(a.tiles_per_group) * ngroups)),
                       dim3(nw * plm::kWave), 0, st, a);
}

bool q4_fast_ok(int64_t K, const void* x, const uint8_t* const* w, int n) {
    if (K % 32 != 0 || !plm::aligned16(x)) return false;
    for (int i = 0; i < n; ++i)
        if (!plm::aligned16(w[i])) return false;
    return true;
}

}  // namespace

// ====================================================================== C ABI

PLM_EXPORT void q4_dequant_to_fp16(const uint8_t* packed, const uint16_t* scales, uint16_t* out_fp16,
                                   int64_t num_channels, int64_t channel_size) {
    plm::clear_error();
    if (!packed || !scales || !out_fp16 || num_channels <= 0 || channel_size <= 0) {
        plm::fail(1, "q4_dequant_to_fp16: null pointer or empty tensor");
        return;
    }
    q4_dequant_launch(packed, scales, out_fp16, num_channels, channel_size, plm::current_stream());
}

PLM_EXPORT int q4_dequant_many_to_fp16(const uint8_t** packed_ptrs, const uint16_t** scale_ptrs, uint16_t** out_ptrs,
                                       const int64_t* num_channels, const int64_t* channel_sizes,
                                       int64_t tensor_count) {
    if (!packed_ptrs || !scale_ptrs || !out_ptrs || !num_channels || !channel_sizes) return plm::fail(1, "null array");
    if (tensor_count <= 0) return plm::fail(2, "tensor_count <= 0");
    hipStream_t st = plm::current_stream();
    for (int64_t t = 0; t < tensor_count; ++t) {
        if (!packed_ptrs[t] || !scale_ptrs[t] || !out_ptrs[t] || num_channels[t] <= 0 || channel_sizes[t] <= 0)
            continue;
        const int code = q4_dequant_launch(packed_ptrs[t], scale_ptrs[t], out_ptrs[t], num_channels[t],
                                           channel_sizes[t], st);
        if (code != 0) return code;
    }
    return 0;
}

PLM_EXPORT int q4_gemv_f16_f32(const uint8_t* packed, const uint16_t* scales, const uint16_t* hidden, float* out,
                               int64_t rows, int64_t cols) {
    if (!packed || !scales || !hidden || !out) return plm::fail(1, "null pointer");
    if (rows <= 0 || cols <= 0) return plm::fail(2, "bad dimensions");
    hipStream_t st = plm::current_stream();
    Q4RowsArgs a;
    std::memset(&a, 0, sizeof(a));
    a.w[0][0] = packed;
    a.s[0][0] = scales;
    a.x = hidden;
    a.out = out;
    a.rows = rows;
    a.K = cols;
    const uint8_t* wl[1] = {packed};
    if (q4_fast_ok(cols, hidden, wl, 1)) {
        launch_q4_rows<8, 1, false, true>(a, 1, st);
    } else {
        hipLaunchKernelGGL(q4_rows_scalar_kernel<true>, dim3(static_cast<unsigned>(plm::ceil_div(rows, 256))),
                           dim3(256), 0, st, a, 1, 1, 0);
    }
    return plm::check_launch("q4 gemv kernel");
}

PLM_EXPORT int q4_moe_selected_forward_u16(const uint16_t* hidden, const uint8_t** gate_packed_ptrs,
                                           const uint16_t** gate_scale_ptrs, const uint8_t** up_packed_ptrs,
                                           const uint16_t** up_scale_ptrs, const uint8_t** down_packed_ptrs,
                                           const uint16_t** down_scale_ptrs, const float* route_weights,
                                           uint16_t* out_fp16, int64_t hidden_size, int64_t intermediate_size,
                                           int64_t selected_count) {
    if (!hidden || !gate_packed_ptrs || !gate_scale_ptrs || !up_packed_ptrs || !up_scale_ptrs || !down_packed_ptrs ||
        !down_scale_ptrs || !route_weights || !out_fp16 || hidden_size <= 0 || intermediate_size <= 0 ||
        selected_count <= 0)
        return plm::fail(1, "null pointer or bad size");
    for (int64_t e = 0; e < selected_count; ++e) {
        if (!gate_packed_ptrs[e] || !gate_scale_ptrs[e] || !up_packed_ptrs[e] || !up_scale_ptrs[e] ||
            !down_packed_ptrs[e] || !down_scale_ptrs[e])
            return plm::fail(3, "null expert pointer");
    }
    if (selected_count > kMaxGroups) return plm::fail(1, "more than %d selected experts", kMaxGroups);
    hipStream_t st = plm::current_stream();
    const int64_t S = selected_count, H = hidden_size, I = intermediate_size;
    float* act = static_cast<float*>(plm::workspace(static_cast<size_t>(S * I) * sizeof(float)));
    if (act == nullptr) return 2;
    // Phase 1, groups of up to kMaxGroups experts.
    std::vector<const uint8_t*> wl;
    for (int64_t e = 0; e < S; ++e) {
        wl.push_back(gate_packed_ptrs[e]);
        wl.push_back(up_packed_ptrs[e]);
    }
    const bool fast1 = q4_fast_ok(H, hidden, wl.data(), static_cast<int>(wl.size()));
    for (int64_t g0 = 0; g0 < S; g0 += kMaxGroups) {
        const int ng = static_cast<int>(std::min<int64_t>(kMaxGroups, S - g0));
        Q4RowsArgs a;
        std::memset(&a, 0, sizeof(a));
        for (int g = 0; g < ng; ++g) {
            a.w[0][g] = gate_packed_ptrs[g0 + g];
            a.s[0][g] = gate_scale_ptrs[g0 + g];
            a.w[1][g] = up_packed_ptrs[g0 + g];
            a.s[1][g] = up_scale_ptrs[g0 + g];
        }
        a.x = hidden;
        a.out = act + g0 * I;
        a.rows = I;
        a.K = H;
        if (fast1) {
            launch_q4_rows<4, 2, true, true>(a, ng, st);
        } else {
            hipLaunchKernelGGL(q4_rows_scalar_kernel<true>,
                               dim3(static_cast<unsigned>(plm::ceil_div(static_cast<int64_t>(ng) * I, 256))), dim3(256),
                               0, st, a, ng, 2, 1);
        }
        const int code = plm::check_launch("q4 gate/up kernel");
        if (code != 0) return code;
    }
    // Phase 2: all selected experts in one pass when they fit.
    std::vector<const uint8_t*> dl(down_packed_ptrs, down_packed_ptrs + S);
    const bool fast2 = q4_fast_ok(I, act, dl.data(), static_cast<int>(S));
    Q4CombineArgs c;
    std::memset(&c, 0, sizeof(c));
    for (int64_t g = 0; g < S; ++g) {
        c.w[g] = down_packed_ptrs[g];
        c.s[g] = down_scale_ptrs[g];
    }
    c.act = act;
    c.route = route_weights;
    c.out_f16 = out_fp16;
    c.rows = H;
    c.K = I;
    c.ngroups = static_cast<int>(S);
    c.cps = static_cast<int>(plm::ceil_div(I / 2, plm::kChunkBytes));
    if (fast2) {
        constexpr int TR = 8;
        const int nw = waves_for(static_cast<int64_t>(c.cps) * S);
        hipLaunchKernelGGL(q4_combine_kernel<TR>, dim3(static_cast<unsigned>(plm::ceil_div(H, TR))),
                           dim3(nw * plm::kWave), 0, st, c);
    } else {
        hipLaunchKernelGGL(q4_combine_scalar_kernel, dim3(static_cast<unsigned>(plm::ceil_div(H, 256))), dim3(256), 0,
                           st, c);
    }
    return plm::check_launch("q4 down/combine kernel");
}
