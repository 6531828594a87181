// Shared host/device helpers of libpocketlm_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "pocketlm_hip.h"

#define PLM_EXPORT extern "C" __attribute__((visibility("default")))

namespace plm {

constexpr int kWave = 64;
// One "chunk" is what a wave streams in one pass along K: 64 lanes x 16 bytes.
constexpr int kChunkBytes = 1024;

// ---------------------------------------------------------------- host side

// Stream used by the calling thread (pocketlm_set_stream).
hipStream_t current_stream();

// Record a failure text for pocketlm_last_error() and return `code`.
int fail(int code, const char* fmt, ...);

// Forget the previous failure text (entry points without a return code).
void clear_error();

// Map a HIP error to the library's return code -(1000 + err) and record it.
int hip_fail(hipError_t err, const char* where);

// Check the last launch; returns 0 or the HIP failure code.
int check_launch(const char* where);

// Device scratch owned by the library, one arena per (device, stream, host
// thread).  The returned block is the arena's until a larger request
// replaces it; replaced blocks are kept, never freed, so launches already
// queued and graphs captured earlier stay valid.  No stream synchronisation,
// so it may run under stream capture.  Returns nullptr on allocation failure
// (after recording the error).
void* workspace(size_t bytes);
// Device words private to the kernels of one (device, stream, host thread),
// zeroed by a kernel on the stream when first handed out and kept until the
// process ends (nothing else writes them), for records that must survive
// other calls' use of the workspace.  Returns nullptr on allocation failure.
constexpr int kStreamWords = 64;
unsigned* stream_words();

// Number of compute units of the current device (cached).
int cu_count();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace plm

// ---------------------------------------------------------------- device side

typedef float plm_float2 __attribute__((ext_vector_type(2)));

// Decode four e4m3fn bytes (one dword, byte 0 first) with the hardware
// converter; NaN bytes (0x7F / 0xFF) come out as NaN.
// A load through the global address space.  Pointers the compiler cannot
// prove global (read from memory, as the device-routed plan's are) would
// otherwise become flat loads, which also count against lgkmcnt: the wait
// for a later scalar load then waits for them too.
typedef uint32_t plm_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 plm_gload16(const void* p) {
    const plm_u32x4 v = *(const __attribute__((address_space(1))) plm_u32x4*)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float plm_gload_f32(const void* p) {
    return *(const __attribute__((address_space(1))) float*)(p);
}

__device__ __forceinline__ void plm_decode4_e4m3(uint32_t d, float* v) {
    const plm_float2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(d), false);
    const plm_float2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(d), true);
    v[0] = lo[0];
    v[1] = lo[1];
    v[2] = hi[0];
    v[3] = hi[1];
}

// Sum across the 64 lanes of a wave with DPP row operations (no LDS
// traffic); the total is valid in lane 63 only.  The addition tree is fixed,
// so a value's sum does not depend on what else the wave reduces or on the
// tile shape a kernel instance uses.
#define PLM_DPP_ADD(v, ctrl, row_mask)                                                                   \
    ((v) + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, (v)), (ctrl), \
                                                                 (row_mask), 0xF, false)))

__device__ __forceinline__ float plm_wave_sum(float v) {
    v = PLM_DPP_ADD(v, 0xB1, 0xF);   // quad_perm [1,0,3,2]: pairs
    v = PLM_DPP_ADD(v, 0x4E, 0xF);   // quad_perm [2,3,0,1]: quads
    v = PLM_DPP_ADD(v, 0x141, 0xF);  // row_half_mirror: groups of 8
    v = PLM_DPP_ADD(v, 0x140, 0xF);  // row_mirror: rows of 16
    v = PLM_DPP_ADD(v, 0x142, 0xA);  // row_bcast:15 into rows 1 and 3
    v = PLM_DPP_ADD(v, 0x143, 0xC);  // row_bcast:31 into rows 2 and 3
    return v;                        // lane 63 holds the wave total
}

constexpr int kSumLane = 63;

__device__ __forceinline__ float plm_silu_mul(float gate, float up) {
    // g / (1 + exp(-g)) * up, all fp32 (fp8_linear.cpp:279-280)
    const float s = gate / (1.0f + expf(-gate));
    return s * up;
}
