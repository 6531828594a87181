// Q4 kernels for gfx950: dequant (src/pcketlm/native/q4_dequant.cpp:171-286),
// the per-row Q4 dot and the fused one-token SwiGLU MoE (357-476).
//
// Format (src/pcketlm/core/model_import/q4_quantize.py:21-71): signed
// two's-complement nibbles flat over the tensor, element 2i in the low
// nibble of byte i, one fp16 scale per channel (row).
//
// Dot products.  A lane reads 16 packed bytes (32 values) per load.  Each
// dword d holds 8 nibbles; u = d ^ 0x88888888 turns every signed nibble q
// into the unsigned u = q + 8, which is unpacked without per-element
// extracts into exact fp16 subnormal pairs: matrix-core operands when x is
// fp16 (gate/up and the plain GEMV), v_fma_mix operands when x is fp32 (the
// down phase).  The +8 bias is removed with sum(q*x) = sum(u*x) - 8*sum(x).
// The row scale multiplies the row's sum.
#include <algorithm>
#include <atomic>
#include <cstring>
#include <vector>

#include "common.h"

namespace {

constexpr int kMaxGroups = 64;

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

// Fast path: channel_size % 32 == 0 (a channel is whole dwords of packed
// data).  A lane converts one packed dword (8 values) into one 16-byte store,
// so each wave-wide store is 1 KB contiguous; a thread handles 4 dwords
// 256 apart, loading all four before converting.
__global__ __launch_bounds__(256) void q4_dequant_kernel(const uint32_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ scales,
                                                         uint4* __restrict__ out, uint32_t ndw,
                                                         uint32_t dw_per_channel) {
    const uint32_t base = blockIdx.x * 1024u + threadIdx.x;
    uint32_t d[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) d[p] = packed[min(base + p * 256u, ndw - 1u)];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t idx = base + p * 256u;
        if (idx >= ndw) break;
        const float sc = h2f_ref(scales[idx / dw_per_channel]);
        const bool finite = (f2u(sc) & 0x7F800000u) != 0x7F800000u;
        uint32_t h[4];
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            // sign-extend nibbles k and k+1
            const float q0 = static_cast<float>(static_cast<int>(d[p] << (28 - 4 * k)) >> 28);
            const float q1 = static_cast<float>(static_cast<int>(d[p] << (24 - 4 * k)) >> 28);
            uint32_t lo, hi;
            if (finite) {
                lo = f16_rne_hw(q0 * sc);
                hi = f16_rne_hw(q1 * sc);
            } else {
                lo = f16_from_bits(q_mul_bits(q0, sc), true);
                hi = f16_from_bits(q_mul_bits(q1, sc), true);
            }
            h[k / 2] = lo | (hi << 16);
        }
        out[idx] = make_uint4(h[0], h[1], h[2], h[3]);
    }
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
    if (cs % 32 == 0 && plm::aligned16(packed) && plm::aligned16(out) && total / 8 < (int64_t{1} << 31)) {
        const int64_t ndw = total / 8;
        hipLaunchKernelGGL(q4_dequant_kernel, dim3(static_cast<unsigned>(plm::ceil_div(ndw, 1024))), dim3(256), 0, st,
                           reinterpret_cast<const uint32_t*>(packed), scales, reinterpret_cast<uint4*>(out),
                           static_cast<uint32_t>(ndw), static_cast<uint32_t>(cs / 8));
    } else {
        hipLaunchKernelGGL(q4_dequant_scalar_kernel, dim3(static_cast<unsigned>(plm::ceil_div(total, 256))),
                           dim3(256), 0, st, packed, scales, out, channels, cs);
    }
    return plm::check_launch("q4 dequant kernel");
}

// ------------------------------------------------------------------ dot products
//
// Layout of the dot-product kernels.  A wave is four groups of 16 lanes; a
// group owns TR rows and reads them in steps of 256 packed bytes (512 values),
// 16 bytes per lane, so one wave-wide load instruction fetches 4 x 256
// contiguous bytes.  The NWS waves of a workgroup split a row's steps, and
// every load is unconditional: rows and steps past the end read a clamped
// address and their contribution is dropped.

typedef _Float16 plm_half2 __attribute__((ext_vector_type(2)));
typedef _Float16 plm_half8 __attribute__((ext_vector_type(8)));
typedef float plm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t plm_u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_lo(uint32_t v) { return static_cast<float>(__builtin_bit_cast(plm_half2, v)[0]); }
__device__ __forceinline__ float half_hi(uint32_t v) { return static_cast<float>(__builtin_bit_cast(plm_half2, v)[1]); }

// sum over a 32-value span of q * x for fp32 x.  Dword i of the span holds
// nibbles k = 0..7 (values 8i + k).  With u = d ^ 0x88888888 (u = q + 8),
// (u >> 4j) & 0x000F000F is the pair (u_{8i+j}, u_{8i+j+4}) as fp16
// subnormals u * 2^-24.  Each product is one fp32 fma (v_fma_mix_f32 reads
// the fp16 half in place, so every product is exact and every add is
// round-to-nearest fp32); 2^24 * sum(u * 2^-24 * x) - 8 * sum(x) is then
// sum(q * x).
__device__ __forceinline__ float q4_span_dot_f32(const uint4& q, const float* x, float xs8) {
    const uint32_t d[4] = {q.x ^ 0x88888888u, q.y ^ 0x88888888u, q.z ^ 0x88888888u, q.w ^ 0x88888888u};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t pr = (d[i] >> (4 * j)) & 0x000F000Fu;
            p = fmaf(half_lo(pr), x[8 * i + j], p);
            p = fmaf(half_hi(pr), x[8 * i + j + 4], p);
        }
    }
    return p * 16777216.0f - xs8;
}

constexpr int kStepBytes = 256;

// Matrix-core dot products for fp16 activations.
//
// v_mfma_f32_16x16x32_f16 is used as a per-lane dot product: lane l supplies
// 8 weights as row l % 16 of A and the 8 matching activations as column l % 16
// of B, so the diagonal D[i][i] is the sum of the own-dot products of the four
// lanes with l % 16 == i (the 240 off-diagonal outputs are cross terms and are
// never read).  Any assignment of k positions to lanes is then valid as long
// as those four lanes share a row: rows are given by (l % 16) / 4 and the 16
// lanes of a row take the 16 pieces of a 256-byte step, the load layout above.
//
// Weights become exact fp16 subnormals: with u = d ^ 0x88888888 (u = q + 8
// per nibble), (u >> 4j) & 0x000F000F is the pair (u_j, u_{j+4}) * 2^-24.  The
// matching B pairs are (x_j, x_{j+4}).  A second accumulator with the
// constant 8 * 2^-24 as A collects 8 * sum(x) on its diagonal, so
// sum(q * x) = 2^24 * (D - C).  Products are exact for every finite fp16 x;
// the matrix core rounds its internal sums, which leaves results within about
// 1e-5 relative of an fp32 FMA chain.
__device__ __forceinline__ plm_half8 q4_mfma_a(uint32_t d) {
    const uint32_t u = d ^ 0x88888888u;
    const plm_u4 r = {u & 0x000F000Fu, (u >> 4) & 0x000F000Fu, (u >> 8) & 0x000F000Fu, (u >> 12) & 0x000F000Fu};
    return __builtin_bit_cast(plm_half8, r);
}

// B for 8 consecutive fp16 activations (x0, x1), (x2, x3), (x4, x5), (x6, x7):
// the pairs (x0, x4), (x1, x5), (x2, x6), (x3, x7).
__device__ __forceinline__ plm_half8 q4_mfma_b(const uint4& v) {
    const plm_u4 r = {__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                      __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
    return __builtin_bit_cast(plm_half8, r);
}

__device__ __forceinline__ plm_half8 q4_mfma_c8() {
    return __builtin_bit_cast(plm_half8, plm_u4{0x00080008u, 0x00080008u, 0x00080008u, 0x00080008u});
}

// Shorter encoding for B values prepared in advance (the down phase): the
// pairs (u1, u5) and (u3, u7) stay in place at bits 4-7 of each half, i.e.
// u * 2^-20, and their B values are stored divided by 16.  Five operations per
// dword: u & 0x000F000F, u & 0x00F000F0, and the same on u >> 8.
__device__ __forceinline__ plm_half8 q4_mfma_a_inplace(uint32_t d) {
    const uint32_t u = d ^ 0x88888888u;
    const uint32_t t = u >> 8;
    const plm_u4 r = {u & 0x000F000Fu, u & 0x00F000F0u, t & 0x000F000Fu, t & 0x00F000F0u};
    return __builtin_bit_cast(plm_half8, r);
}

__device__ __forceinline__ plm_half8 q4_mfma_c8_inplace() {
    return __builtin_bit_cast(plm_half8, plm_u4{0x00080008u, 0x00800080u, 0x00080008u, 0x00800080u});
}

// The down phase reads its fp32 activations as two fp16 planes already in
// the B operand order: for value k, step s = k / 512, piece p = (k / 32) % 16,
// dword j = (k / 8) % 4 and n = k % 8, the uint4 ((s * 4 + j) * 2 + plane) * 16
// + p holds it in half (n % 4) * 2 + n / 4.  Values with n % 4 odd are stored
// divided by 16: the down kernel's weights use the shorter encoding below,
// which leaves those nibbles 16 times too large.  With v' the stored value,
// plane 0 is hi = fp16(v') and plane 1 is lo = fp16((v' - hi) * 2^11), so
// hi + lo * 2^-11 carries 22 significant bits (the split follows the /16, so
// no bits are lost to it).  A value that fp16 cannot hold (|v| >= 65504, inf,
// NaN) records the call's number in a word private to the stream and host
// thread, and that call's down phase reads the fp32 activations instead.
// The call's number is one more than an epoch word kept in device memory
// beside the record: after a call that recorded its number, the down phase's
// last workgroup advances the epoch, so the next call (or replay of a
// captured graph) has a new number without the host, and at the start of
// every call the record is at most the epoch, which selects nothing.  Calls
// that record nothing touch neither word (no atomics on the common path).
// Words: [0] epoch, [1] record, [2] the down phase's finished-workgroup
// count.
constexpr int kQ4Epoch = 0, kQ4Record = 1, kQ4Done = 2;

__device__ __forceinline__ void q4_store_planes(uint4* base, int64_t k, float v, unsigned* words) {
    if (!(fabsf(v) < 65504.0f))
        atomicExch(words + kQ4Record,
                   __hip_atomic_load(words + kQ4Epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u);
    const int64_t s = k >> 9;
    const int p = static_cast<int>((k >> 5) & 15), j = static_cast<int>((k >> 3) & 3), n = static_cast<int>(k & 7);
    const float vs = (n & 1) ? v * 0.0625f : v;
    const _Float16 hi = static_cast<_Float16>(vs);
    const _Float16 lo = static_cast<_Float16>((vs - static_cast<float>(hi)) * 2048.0f);
    uint16_t* h = reinterpret_cast<uint16_t*>(base + ((s * 4 + j) * 2) * 16 + p) + (n & 3) * 2 + (n >> 2);
    h[0] = __builtin_bit_cast(uint16_t, hi);
    h[16 * 8] = __builtin_bit_cast(uint16_t, lo);  // plane 1: 16 uint4 further
}

struct Q4RowsArgs {
    const uint8_t* w[2][kMaxGroups];
    const uint16_t* s[2][kMaxGroups];
    const void* x;        // fp16 or fp32 activations [K]
    float* out;           // (g, row) at g * out_stride + row, or the step order below
    int64_t rows;
    int64_t K;            // values per row (multiple of 32 on this path)
    int64_t out_stride;
    int out_steps;        // write the output in step order (see act_pos)
    int tiles_per_group;
    uint4* planes;        // SILU only: also write the fp16 B planes (nullptr: no)
    int64_t planes_stride;  // uint4 per group
    unsigned* words;      // epoch and overflow record (with planes)
};

// Position of value k of an fp32 activation vector stored in "step order":
// within each 512-value step, value li * 32 + e (the e-th value of lane li's
// 16-byte weight span) sits at (e / 4) * 64 + li * 4 + e % 4, so that the
// i-th float4 load of the 16 lanes of a row group reads 256 contiguous
// bytes.  The buffer is padded to whole steps.
__device__ __forceinline__ int64_t act_pos(int64_t k) {
    return (k & ~int64_t{511}) | (((k & 31) >> 2) << 6) | (((k & 511) >> 5) << 2) | (k & 3);
}

// Rows of one or more experts against one shared fp16 activation vector, on
// the matrix cores.  NWT=2 with SILU computes silu(gate) * up (the gate/up
// phase of the MoE).
// The 16-wave long-row GEMV fits in 64 VGPRs, so it asks for 8 waves per
// SIMD (two workgroups per CU): 10.1 -> 9.7 us on 3584 x 18944.  The others
// would spill at that bound.
template <int NWS>
constexpr int q4_rows_min_waves() {
    return NWS >= 16 ? 8 : 1;
}

template <int TR, int NWT, int NWS, bool SILU>
__global__ __launch_bounds__(NWS * 64, q4_rows_min_waves<NWS>()) void q4_rows_kernel(const Q4RowsArgs a) {
    constexpr int T = 4 * TR;  // rows per workgroup
    __shared__ float red[NWS][NWT][T];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, c = i16 >> 2;
    const int piece = (i16 & 3) + 4 * (lane >> 4);  // 16-byte piece of the step
    const int g = blockIdx.x / a.tiles_per_group;
    const int64_t tile0 = static_cast<int64_t>(blockIdx.x - g * a.tiles_per_group) * T;
    const int64_t row_bytes = a.K >> 1;
    const int steps = static_cast<int>((row_bytes + kStepBytes - 1) / kStepBytes);
    const uint8_t* wp[NWT];
    int64_t roff[TR];
#pragma unroll
    for (int i = 0; i < NWT; ++i) wp[i] = a.w[i][g];
#pragma unroll
    for (int t = 0; t < TR; ++t) {
        const int64_t row = tile0 + c * TR + t;
        roff[t] = (row < a.rows ? row : a.rows - 1) * row_bytes;
    }
    plm_f4 acc[NWT][TR], corr = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NWT; ++i)
#pragma unroll
        for (int t = 0; t < TR; ++t) acc[i][t] = plm_f4{0.0f, 0.0f, 0.0f, 0.0f};
    const plm_half8 c8 = q4_mfma_c8();

    for (int s = wave; s < steps; s += NWS) {
        const int64_t byte = static_cast<int64_t>(s) * kStepBytes + piece * 16;
        const bool ok = byte < row_bytes;
        const int64_t bc = ok ? byte : row_bytes - 16;
        uint4 q[NWT][TR];
#pragma unroll
        for (int i = 0; i < NWT; ++i)
#pragma unroll
            for (int t = 0; t < TR; ++t) q[i][t] = *reinterpret_cast<const uint4*>(wp[i] + roff[t] + bc);
        const uint4* xp = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.x) + 2 * bc);
        uint4 xv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) xv[k] = xp[k];
        if (!ok) {
            // a piece past the end of the row contributes nothing
#pragma unroll
            for (int k = 0; k < 4; ++k) xv[k] = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const plm_half8 b = q4_mfma_b(xv[j]);
            corr = __builtin_amdgcn_mfma_f32_16x16x32_f16(c8, b, corr, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < NWT; ++i)
#pragma unroll
                for (int t = 0; t < TR; ++t) {
                    const uint32_t d = j == 0 ? q[i][t].x : j == 1 ? q[i][t].y : j == 2 ? q[i][t].z : q[i][t].w;
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(q4_mfma_a(d), b, acc[i][t], 0, 0, 0);
                }
        }
    }

    // D[i][i] sits in lane 16 * (i / 4) + i, element i % 4; row group c owns
    // i = 4c .. 4c + 3, i.e. the aligned quad of lanes 20c .. 20c + 3, each
    // contributing its element lane % 4.
    const int e = lane & 3;
    const float cr = corr[e];
#pragma unroll
    for (int i = 0; i < NWT; ++i)
#pragma unroll
        for (int t = 0; t < TR; ++t) {
            float v = acc[i][t][e] - cr;
            v = PLM_DPP_ADD(v, 0xB1, 0xF);
            v = PLM_DPP_ADD(v, 0x4E, 0xF);
            if (lane == 20 * c) red[wave][i][c * TR + t] = v;
        }
    __syncthreads();
    if (threadIdx.x < T) {
        const int64_t row = tile0 + threadIdx.x;
        if (row < a.rows) {
            float v[NWT];
#pragma unroll
            for (int i = 0; i < NWT; ++i) {
                float sum = 0.0f;
#pragma unroll
                for (int w = 0; w < NWS; ++w) sum += red[w][i][threadIdx.x];
                v[i] = sum * 16777216.0f * h2f_ref(a.s[i][g][row]);
            }
            const int64_t o = static_cast<int64_t>(g) * a.out_stride + (a.out_steps ? act_pos(row) : row);
            if constexpr (SILU) {
                const float act = plm_silu_mul(v[0], v[1]);
                a.out[o] = act;
                if (a.planes != nullptr) q4_store_planes(a.planes + g * a.planes_stride, row, act, a.words);
            } else {
                a.out[o] = v[0];
            }
        }
    }
}

struct Q4CombineArgs {
    const uint8_t* w[kMaxGroups];
    const uint16_t* s[kMaxGroups];
    const float* act;     // [ngroups][act_stride] fp32, step order (act_pos) on the fast path
    int64_t act_stride;
    const uint4* planes;  // [ngroups][planes_stride] fp16 B planes, or nullptr
    int64_t planes_stride;
    unsigned* words;      // epoch, overflow record, finished count (with planes)
    const float* route;   // [ngroups]
    uint16_t* out_f16;    // [rows]
    int64_t rows;
    int64_t K;
    int ngroups;
};

// Down phase + routed combine of the Q4 MoE, fp16 out (software RNE).  The
// (expert, step) items are split over the waves in expert order; a wave sums
// the steps of one expert raw and folds that sum into the output with the
// expert's row scale and route weight when its expert changes.  Lanes are
// laid out as in q4_rows_kernel.  The activations come from the fp16 planes
// on the matrix cores, or from the fp32 vector with v_fma_mix when the planes
// are absent or could not hold this call's values.
template <int TR, int NWS>
__global__ __launch_bounds__(NWS * 64) void q4_down_kernel(const Q4CombineArgs a) {
    constexpr int T = 4 * TR;
    __shared__ float red[NWS][T];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, c = i16 >> 2;
    const int piece = (i16 & 3) + 4 * (lane >> 4);
    const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * T;
    const int64_t row_bytes = a.K >> 1;
    const int steps = static_cast<int>((row_bytes + kStepBytes - 1) / kStepBytes);
    const int ng = a.ngroups;
    int64_t rc[TR], roff[TR];
#pragma unroll
    for (int t = 0; t < TR; ++t) {
        const int64_t row = tile0 + c * TR + t;
        rc[t] = row < a.rows ? row : a.rows - 1;
        roff[t] = rc[t] * row_bytes;
    }
    float tot[TR];
#pragma unroll
    for (int t = 0; t < TR; ++t) tot[t] = 0.0f;

    // The wave's items are (expert g, step s) = wave, wave + NWS, ... in the
    // order g * steps + s; the walk advances (g, s) without a division and
    // reloads an expert's pointers only when the expert changes.
    int g = 0, s = wave;
    while (g < ng && s >= steps) {
        s -= steps;
        ++g;
    }
    auto advance = [&]() {
        s += NWS;
        while (s >= steps) {
            s -= steps;
            ++g;
        }
    };
    const int gl = g < ng ? g : ng - 1;  // a wave without items reads a valid address and stops below
    const uint8_t* wg = a.w[gl];
    uint4 q[TR];
    auto load_w = [&](int step) {
        const int64_t byte = static_cast<int64_t>(step) * kStepBytes + piece * 16;
        const int64_t bc = byte < row_bytes ? byte : row_bytes - 16;
#pragma unroll
        for (int t = 0; t < TR; ++t) q[t] = *reinterpret_cast<const uint4*>(wg + roff[t] + bc);
    };
    // Keeps each path's weight arithmetic inside its branch (otherwise the
    // compiler hoists the shared part above the branch and waits for the
    // weights before the record is read).  Placed after each path's
    // activation loads, so it never delays them.
    auto pin_w = [&]() {
#pragma unroll
        for (int t = 0; t < TR; ++t) asm volatile("" : "+v"(q[t].x), "+v"(q[t].y), "+v"(q[t].z), "+v"(q[t].w));
    };
    // Both paths read the same weights: the first item's go out right after
    // the overflow record's read, which hides that read's latency.
    const unsigned flagged =
        a.planes != nullptr ? __hip_atomic_load(a.words + kQ4Record, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
    const unsigned epoch =
        a.planes != nullptr ? __hip_atomic_load(a.words + kQ4Epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
    load_w(g < ng ? s : steps - 1);
    const bool use_planes =
        a.planes != nullptr && __builtin_amdgcn_readfirstlane(flagged) != __builtin_amdgcn_readfirstlane(epoch) + 1u;

    if (use_planes) {
        plm_f4 ah[TR], al[TR], ch = {0.0f, 0.0f, 0.0f, 0.0f}, cl = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < TR; ++t) ah[t] = al[t] = plm_f4{0.0f, 0.0f, 0.0f, 0.0f};
        const plm_half8 c8 = q4_mfma_c8_inplace();
        const int e = lane & 3;
        auto fold = [&](int ge) {
            const float rw = a.route[ge] * 16777216.0f;
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                const float v = (ah[t][e] - ch[e]) + (al[t][e] - cl[e]) * (1.0f / 2048.0f);
                tot[t] = fmaf(v * h2f_ref(a.s[ge][rc[t]]), rw, tot[t]);
                ah[t] = al[t] = plm_f4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            ch = cl = plm_f4{0.0f, 0.0f, 0.0f, 0.0f};
        };
        // Two items in flight: the next item's weights and B values are read
        // before the current one is computed (an item past the last re-reads
        // the current one's addresses; its values are not used).
        const uint4* pg = a.planes + static_cast<int64_t>(gl) * a.planes_stride;
        uint4 bv[8];
        auto load_b = [&](const uint4* pgx, int step, uint4 (&dst)[8]) {
            const uint4* bp = pgx + static_cast<int64_t>(step) * 128 + piece;
#pragma unroll
            for (int k = 0; k < 8; ++k) dst[k] = bp[k * 16];
        };
        load_b(pg, g < ng ? s : steps - 1, bv);
        while (g < ng) {
            int gn = g, sn = s;
            sn += NWS;
            while (sn >= steps) {
                sn -= steps;
                ++gn;
            }
            const int gq = gn < ng ? gn : g, sq = gn < ng ? sn : s;
            const uint8_t* wn = a.w[gq];
            const uint4* pn = a.planes + static_cast<int64_t>(gq) * a.planes_stride;
            uint4 qn[TR], bn[8];
            {
                const int64_t byte = static_cast<int64_t>(sq) * kStepBytes + piece * 16;
                const int64_t bc = byte < row_bytes ? byte : row_bytes - 16;
#pragma unroll
                for (int t = 0; t < TR; ++t) qn[t] = *reinterpret_cast<const uint4*>(wn + roff[t] + bc);
            }
            load_b(pn, sq, bn);
            const bool ok = static_cast<int64_t>(s) * kStepBytes + piece * 16 < row_bytes;
            if (!ok) {
#pragma unroll
                for (int k = 0; k < 8; ++k) bv[k] = make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const plm_half8 bh = __builtin_bit_cast(plm_half8, bv[2 * j]);
                const plm_half8 bl = __builtin_bit_cast(plm_half8, bv[2 * j + 1]);
                ch = __builtin_amdgcn_mfma_f32_16x16x32_f16(c8, bh, ch, 0, 0, 0);
                cl = __builtin_amdgcn_mfma_f32_16x16x32_f16(c8, bl, cl, 0, 0, 0);
#pragma unroll
                for (int t = 0; t < TR; ++t) {
                    const uint32_t d = j == 0 ? q[t].x : j == 1 ? q[t].y : j == 2 ? q[t].z : q[t].w;
                    const plm_half8 av = q4_mfma_a_inplace(d);
                    ah[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh, ah[t], 0, 0, 0);
                    al[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl, al[t], 0, 0, 0);
                }
            }
            if (gn != g) fold(g);
            g = gn;
            s = sn;
#pragma unroll
            for (int t = 0; t < TR; ++t) q[t] = qn[t];
#pragma unroll
            for (int k = 0; k < 8; ++k) bv[k] = bn[k];
        }
        // the diagonal elements of row group c sit in the quad 20c .. 20c + 3
#pragma unroll
        for (int t = 0; t < TR; ++t) {
            tot[t] = PLM_DPP_ADD(tot[t], 0xB1, 0xF);
            tot[t] = PLM_DPP_ADD(tot[t], 0x4E, 0xF);
        }
    } else {
        float part[TR];
#pragma unroll
        for (int t = 0; t < TR; ++t) part[t] = 0.0f;
        auto fold = [&](int ge) {
            const float rw = a.route[ge];
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                tot[t] = fmaf(part[t] * h2f_ref(a.s[ge][rc[t]]), rw, tot[t]);
                part[t] = 0.0f;
            }
        };
        const float* ag = a.act + static_cast<int64_t>(gl) * a.act_stride;
        bool first = true;
        while (g < ng) {
            if (!first) load_w(s);
            first = false;
            const bool ok = static_cast<int64_t>(s) * kStepBytes + piece * 16 < row_bytes;
            // step order: the i-th float4 of piece p is at step * 512 + i * 64 + p * 4
            const float4* xp = reinterpret_cast<const float4*>(ag + static_cast<int64_t>(s) * 512 + piece * 4);
            float4 xv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = xp[i * 16];
            pin_w();
            float x[32], xs = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x[4 * i] = xv[i].x;
                x[4 * i + 1] = xv[i].y;
                x[4 * i + 2] = xv[i].z;
                x[4 * i + 3] = xv[i].w;
                xs += xv[i].x + xv[i].y + xv[i].z + xv[i].w;
            }
#pragma unroll
            for (int t = 0; t < TR; ++t) {
                const float p = q4_span_dot_f32(q[t], x, 8.0f * xs);
                part[t] += ok ? p : 0.0f;
            }
            const int gprev = g;
            advance();
            if (g != gprev) {
                fold(gprev);
                if (g < ng) {
                    wg = a.w[g];
                    ag = a.act + static_cast<int64_t>(g) * a.act_stride;
                }
            }
        }
        // row group c is the 16 lanes with (lane % 16) / 4 == c
#pragma unroll
        for (int t = 0; t < TR; ++t) {
            float v = tot[t];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            v = PLM_DPP_ADD(v, 0xB1, 0xF);
            tot[t] = PLM_DPP_ADD(v, 0x4E, 0xF);
        }
    }
    if (lane == 20 * c) {
#pragma unroll
        for (int t = 0; t < TR; ++t) red[wave][c * TR + t] = tot[t];
    }
    __syncthreads();
    if (threadIdx.x < T) {
        const int64_t row = tile0 + threadIdx.x;
        if (row < a.rows) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < NWS; ++w) v += red[w][threadIdx.x];
            a.out_f16[row] = f16_from_bits(f2u(v), false);
        }
    }
    // After a flagged call the last workgroup to finish advances the epoch,
    // so the record (this call's number) never matches a later call.  Every
    // workgroup read the record and the epoch (the values decide this
    // branch) before it counts itself; a call that flagged nothing leaves
    // both words as they are, the record staying at most the epoch.  The
    // kernel's end makes the new epoch visible to the next call.
    if (a.planes != nullptr && !use_planes && threadIdx.x == 0) {
        const unsigned done =
            __hip_atomic_fetch_add(a.words + kQ4Done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == gridDim.x - 1) {
            __hip_atomic_store(a.words + kQ4Done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(a.words + kQ4Epoch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    a.out[static_cast<int64_t>(g) * a.out_stride + (a.out_steps ? act_pos(row) : row)] =
        silu ? plm_silu_mul(v[0], v[1]) : v[0];
}

__global__ void q4_combine_scalar_kernel(const Q4CombineArgs a) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= a.rows) return;
    float acc = 0.0f;
    for (int g = 0; g < a.ngroups; ++g) {
        float s = 0.0f;
        for (int64_t k = 0; k < a.K; ++k)
            s = fmaf(static_cast<float>(q4_at(a.w[g], row * a.K + k)), a.act[static_cast<int64_t>(g) * a.act_stride + k], s);
        acc = fmaf(s * h2f_ref(a.s[g][row]), a.route[g], acc);
    }
    a.out_f16[row] = f16_from_bits(f2u(acc), false);
}

template <int TR, int NWT, int NWS, bool SILU>
void launch_q4_rows(Q4RowsArgs a, int ngroups, hipStream_t st) {
    a.tiles_per_group = static_cast<int>(plm::ceil_div(a.rows, 4 * TR));
    hipLaunchKernelGGL((q4_rows_kernel<TR, NWT, NWS, SILU>),
                       dim3(static_cast<unsigned>(static_cast<int64_t>(a.tiles_per_group) * ngroups)),
                       dim3(NWS * plm::kWave), 0, st, a);
}

// Long rows (many 256-byte steps) favour fewer rows per group and more
// waves splitting each row; short rows the opposite.
void launch_q4_gemv(const Q4RowsArgs& a, hipStream_t st) {
    if (a.K / 2 >= 16 * kStepBytes) {
        launch_q4_rows<2, 1, 16, false>(a, 1, st);
    } else {
        launch_q4_rows<4, 1, 4, false>(a, 1, st);
    }
}

// The vector kernels need whole 16-byte spans: K % 32 == 0 and 16-byte
// aligned weight (and activation) pointers.
bool q4_weights_ok(int64_t K, const uint8_t* const* w, int n) {
    if (K % 32 != 0) return false;
    for (int i = 0; i < n; ++i)
        if (!plm::aligned16(w[i])) return false;
    return true;
}

bool q4_fast_ok(int64_t K, const void* x, const uint8_t* const* w, int n) {
    return plm::aligned16(x) && q4_weights_ok(K, w, n);
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
    a.out_stride = rows;
    const uint8_t* wl[1] = {packed};
    if (q4_fast_ok(cols, hidden, wl, 1)) {
        launch_q4_gemv(a, st);
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
    std::vector<const uint8_t*> dl(down_packed_ptrs, down_packed_ptrs + S);
    // The down kernel's fast path reads the activations in step order, padded
    // to whole 512-value steps; the plain layout otherwise.  The workspace is
    // 256-byte aligned, so only the down weights and I decide.
    const bool fast2 = q4_weights_ok(I, dl.data(), static_cast<int>(S));
    const int64_t stride = fast2 ? plm::ceil_div(I, 512) * 512 : I;
    std::vector<const uint8_t*> wl;
    for (int64_t e = 0; e < S; ++e) {
        wl.push_back(gate_packed_ptrs[e]);
        wl.push_back(up_packed_ptrs[e]);
    }
    const bool fast1 = q4_fast_ok(H, hidden, wl.data(), static_cast<int>(wl.size()));
    // With both fast paths the gate/up kernel also writes the activations as
    // fp16 B planes for the matrix-core down phase (same size as the fp32
    // vector, after it in the workspace).
    const bool planes = fast1 && fast2;
    const int64_t planes_stride = stride / 4;  // uint4 per expert
    // The epoch and overflow record live in the stream's private words
    // (written by nothing else); the workspace, which other entry points on
    // the stream reuse, holds [fp32 act][planes].
    unsigned* words = plm::stream_words();
    if (words == nullptr) return 2;
    char* ws = static_cast<char*>(plm::workspace(static_cast<size_t>(S * stride) * sizeof(float) * (planes ? 2 : 1)));
    if (ws == nullptr) return 2;
    float* act = reinterpret_cast<float*>(ws);
    uint4* bplanes = planes ? reinterpret_cast<uint4*>(act + S * stride) : nullptr;
    // Phase 1, groups of up to kMaxGroups experts.
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
        a.out = act + g0 * stride;
        a.rows = I;
        a.K = H;
        a.out_stride = stride;
        a.out_steps = fast2 ? 1 : 0;
        a.planes = planes ? bplanes + g0 * planes_stride : nullptr;
        a.planes_stride = planes_stride;
        a.words = words;
        if (fast1) {
            launch_q4_rows<2, 2, 4, true>(a, ng, st);
        } else {
            hipLaunchKernelGGL(q4_rows_scalar_kernel<true>,
                               dim3(static_cast<unsigned>(plm::ceil_div(static_cast<int64_t>(ng) * I, 256))), dim3(256),
                               0, st, a, ng, 2, 1);
        }
        const int code = plm::check_launch("q4 gate/up kernel");
        if (code != 0) return code;
    }
    // Phase 2: all selected experts in one pass.
    Q4CombineArgs c;
    std::memset(&c, 0, sizeof(c));
    for (int64_t g = 0; g < S; ++g) {
        c.w[g] = down_packed_ptrs[g];
        c.s[g] = down_scale_ptrs[g];
    }
    c.act = act;
    c.act_stride = stride;
    c.planes = bplanes;
    c.planes_stride = planes_stride;
    c.words = words;
    c.route = route_weights;
    c.out_f16 = out_fp16;
    c.rows = H;
    c.K = I;
    c.ngroups = static_cast<int>(S);
    if (fast2) {
        // 4 rows per lane group: each lane's activation read feeds four rows.
        hipLaunchKernelGGL((q4_down_kernel<4, 8>), dim3(static_cast<unsigned>(plm::ceil_div(H, 16))),
                           dim3(8 * plm::kWave), 0, st, c);
    } else {
        hipLaunchKernelGGL(q4_combine_scalar_kernel, dim3(static_cast<unsigned>(plm::ceil_div(H, 256))), dim3(256), 0,
                           st, c);
    }
    return plm::check_launch("q4 down/combine kernel");
}
