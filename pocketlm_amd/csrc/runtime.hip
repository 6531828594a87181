// Runtime plumbing of libpocketlm_hip.so: per-thread stream, error text,
// device probes and the per-(device, stream) scratch arena.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "common.h"

namespace plm {

namespace {

thread_local hipStream_t t_stream = nullptr;
thread_local char t_error[512] = {0};

struct Arena {
    void* ptr = nullptr;
    size_t size = 0;
};

std::mutex g_arena_mu;
std::map<std::pair<int, hipStream_t>, Arena> g_arenas;
std::map<std::pair<int, hipStream_t>, unsigned*> g_words;

}  // namespace

hipStream_t current_stream() { return t_stream; }

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_error, sizeof(t_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { t_error[0] = 0; }

int hip_fail(hipError_t err, const char* where) {
    return fail(-(1000 + static_cast<int>(err)), "%s: %s", where, hipGetErrorString(err));
}

int check_launch(const char* where) {
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return hip_fail(err, where);
    }
    return 0;
}

void* workspace(size_t bytes) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) {
        hip_fail(err, "hipGetDevice");
        return nullptr;
    }
    if (bytes == 0) bytes = 256;
    std::lock_guard<std::mutex> lock(g_arena_mu);
    Arena& a = g_arenas[{dev, t_stream}];
    if (a.size >= bytes) {
        return a.ptr;
    }
    if (a.ptr != nullptr) {
        // Work already queued on this stream may still use the old block.
        err = hipStreamSynchronize(t_stream);
        if (err != hipSuccess) {
            hip_fail(err, "hipStreamSynchronize(workspace)");
            return nullptr;
        }
        hipFree(a.ptr);
        a.ptr = nullptr;
        a.size = 0;
    }
    // Round up to 1 MiB so that small growth does not reallocate each call.
    const size_t rounded = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
    err = hipMalloc(&a.ptr, rounded);
    if (err != hipSuccess) {
        a.ptr = nullptr;
        hip_fail(err, "hipMalloc(workspace)");
        return nullptr;
    }
    a.size = rounded;
    return a.ptr;
}

unsigned* stream_words() {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) {
        hip_fail(err, "hipGetDevice");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_arena_mu);
    unsigned*& w = g_words[{dev, t_stream}];
    if (w == nullptr) {
        void* p = nullptr;
        err = hipMalloc(&p, kStreamWords * sizeof(unsigned));
        if (err == hipSuccess) err = hipMemsetAsync(p, 0, kStreamWords * sizeof(unsigned), t_stream);
        if (err != hipSuccess) {
            if (p != nullptr) hipFree(p);
            hip_fail(err, "stream words");
            return nullptr;
        }
        w = static_cast<unsigned*>(p);
    }
    return w;
}

int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0) {
            n = 256;
        }
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace plm

PLM_EXPORT int pocketlm_set_stream(void* hip_stream) {
    plm::t_stream = static_cast<hipStream_t>(hip_stream);
    return 0;
}

PLM_EXPORT const char* pocketlm_last_error(void) { return plm::t_error; }

PLM_EXPORT int pocketlm_device_available(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

PLM_EXPORT int fp8_dequant_cpu_has_avx2_f16c(void) { return pocketlm_device_available(); }
PLM_EXPORT int fp8_linear_avx512_cpu_has_avx512(void) { return pocketlm_device_available(); }
PLM_EXPORT int q4_cpu_has_avx2_f16c(void) { return pocketlm_device_available(); }
PLM_EXPORT int ds_cpu_has_avx2(void) { return pocketlm_device_available(); }
