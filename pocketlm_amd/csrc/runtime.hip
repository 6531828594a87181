// Runtime plumbing of libpocketlm_hip.so: per-thread stream, error text,
// device probes and the per-(device, stream, host thread) scratch arena.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "common.h"

namespace plm {

namespace {

thread_local hipStream_t t_stream = nullptr;
thread_local char t_error[512] = {0};

// Scratch of one (device, stream) for the calling host thread.  Blocks are
// kept until the thread calls pocketlm_release_scratch (or the process
// ends): a launch already queued, or a HIP graph captured earlier, may still
// read a block that a larger request has since replaced, so growth allocates
// a new block and keeps the old one.  Capacity grows at least twofold, which
// bounds the retired blocks to the size of the current one.  Per thread: two
// host threads enqueueing on one stream interleave their launches, and must
// not share intermediates.
struct Arena {
    void* ptr = nullptr;
    size_t size = 0;
};

struct Words {
    unsigned* ptr = nullptr;
    bool owned = false;  // allocated (a slot of the zeroed pool otherwise)
};

struct ThreadScratch {
    std::map<std::pair<int, hipStream_t>, Arena> arenas;
    std::map<std::pair<int, hipStream_t>, Words> words;
    std::vector<std::pair<int, void*>> retired;  // (device, block) replaced by growth
    size_t bytes = 0;                            // device bytes held (arenas and retired)
};

thread_local ThreadScratch t_scratch;

// Stream words come from a pool that is zero when the module loads, one
// slot per (device, stream, host thread), never handed out twice: no
// zeroing launch is needed, so a first call under stream capture finds its
// words zero both in the graph and outside it.  Past the pool, words are
// allocated and zeroed by a kernel on the stream.
constexpr int kWordSlots = 1024;
__device__ unsigned g_word_pool[kWordSlots * kStreamWords];
std::mutex g_pool_mu;
std::map<int, std::pair<unsigned*, int>> g_pool_next;  // device -> (pool address, next free slot)

// hipMalloc with the calling thread's stream-capture mode relaxed for the
// call: under a capture in the global mode the runtime refuses allocations
// (and invalidates the capture), although the block is an ordinary
// allocation that outlives the graph, which is what the arena needs.
hipError_t malloc_relaxed(void** p, size_t bytes) {
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const hipError_t xe = hipThreadExchangeStreamCaptureMode(&mode);
    const hipError_t err = hipMalloc(p, bytes);
    if (xe == hipSuccess) hipThreadExchangeStreamCaptureMode(&mode);
    return err;
}

__global__ void zero_words_kernel(unsigned* w, int n) {
    const int i = static_cast<int>(threadIdx.x);
    if (i < n) w[i] = 0u;
}

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
    Arena& a = t_scratch.arenas[{dev, t_stream}];
    if (a.size >= bytes) return a.ptr;
    // Round up to 1 MiB, and at least double, so that growth is rare.
    size_t want = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
    if (want < 2 * a.size) want = 2 * a.size;
    void* p = nullptr;
    err = malloc_relaxed(&p, want);
    if (err != hipSuccess) {
        hip_fail(err, "hipMalloc(workspace)");
        return nullptr;
    }
    if (a.ptr != nullptr) t_scratch.retired.emplace_back(dev, a.ptr);
    a.ptr = p;
    a.size = want;
    t_scratch.bytes += want;
    return a.ptr;
}

unsigned* stream_words() {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) {
        hip_fail(err, "hipGetDevice");
        return nullptr;
    }
    Words& slot = t_scratch.words[{dev, t_stream}];
    if (slot.ptr == nullptr) {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        auto it = g_pool_next.find(dev);
        if (it == g_pool_next.end()) {
            void* base = nullptr;
            err = hipGetSymbolAddress(&base, HIP_SYMBOL(g_word_pool));
            if (err != hipSuccess) {
                hip_fail(err, "hipGetSymbolAddress(g_word_pool)");
                return nullptr;
            }
            it = g_pool_next.emplace(dev, std::make_pair(static_cast<unsigned*>(base), 0)).first;
        }
        if (it->second.second < kWordSlots) {
            slot.ptr = it->second.first + static_cast<size_t>(it->second.second) * kStreamWords;
            ++it->second.second;
        }
    }
    unsigned*& w = slot.ptr;
    if (w == nullptr) {
        void* p = nullptr;
        err = malloc_relaxed(&p, kStreamWords * sizeof(unsigned));
        if (err != hipSuccess) {
            hip_fail(err, "stream words");
            return nullptr;
        }
        // zeroed by a kernel on the stream (a captured graph then zeroes them
        // on each replay, before its first use of them)
        hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(kStreamWords), 0, t_stream, static_cast<unsigned*>(p),
                           kStreamWords);
        err = hipGetLastError();
        if (err != hipSuccess) {
            hipFree(p);
            hip_fail(err, "stream words");
            return nullptr;
        }
        w = static_cast<unsigned*>(p);
        slot.owned = true;
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

// Device bytes of scratch the calling host thread holds (its arenas and the
// blocks they replaced).
PLM_EXPORT int64_t pocketlm_scratch_bytes(void) { return static_cast<int64_t>(plm::t_scratch.bytes); }

// Waits for the calling thread's streams, then frees its scratch: arenas,
// the blocks they replaced and allocated stream words (pool slots are not
// handed out again).  Graphs captured by this thread must not be replayed
// afterwards.  The next call on the thread starts a new arena.
PLM_EXPORT int pocketlm_release_scratch(void) {
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return plm::fail(-1, "hipGetDevice failed");
    int code = 0;
    auto on_device = [&](int dev) {
        const hipError_t err = hipSetDevice(dev);
        if (err != hipSuccess && code == 0) code = plm::hip_fail(err, "hipSetDevice");
        return err == hipSuccess;
    };
    for (auto& kv : plm::t_scratch.arenas)
        if (on_device(kv.first.first)) {
            const hipError_t err = hipStreamSynchronize(kv.first.second);
            if (err != hipSuccess && code == 0) code = plm::hip_fail(err, "hipStreamSynchronize");
        }
    for (auto& kv : plm::t_scratch.words)
        if (on_device(kv.first.first)) {
            const hipError_t err = hipStreamSynchronize(kv.first.second);
            if (err != hipSuccess && code == 0) code = plm::hip_fail(err, "hipStreamSynchronize");
        }
    if (code != 0) {
        hipSetDevice(prev);
        return code;  // nothing freed: the streams' work may still read it
    }
    for (auto& kv : plm::t_scratch.arenas)
        if (kv.second.ptr != nullptr && on_device(kv.first.first)) hipFree(kv.second.ptr);
    for (auto& r : plm::t_scratch.retired)
        if (on_device(r.first)) hipFree(r.second);
    for (auto& kv : plm::t_scratch.words)
        if (kv.second.owned && on_device(kv.first.first)) hipFree(kv.second.ptr);
    plm::t_scratch.arenas.clear();
    plm::t_scratch.retired.clear();
    plm::t_scratch.words.clear();
    plm::t_scratch.bytes = 0;
    hipSetDevice(prev);
    return code;
}

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
