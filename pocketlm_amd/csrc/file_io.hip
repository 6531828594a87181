// Weight files to HBM.  The reference reads its on-disk artifacts into host
// memory: FP8 pack spans through mmap (src/pcketlm/core/runtime/fp8_pack.py:
// 54-241), row8 artifacts through fread or a file mapping
// (src/pcketlm/native/row8_artifact_cache.cpp:20-147), Q4 shards through
// safetensors.  Here a file's byte ranges go straight to device memory:
// reader threads pread chunks into pinned staging buffers, and each chunk is
// copied with hipMemcpyAsync on the thread's own stream while the thread
// reads the next one, so page-cache reads and PCIe transfers overlap and
// several DMA queues run at once.
//
// Host code only (no kernels).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "common.h"

namespace {

constexpr size_t kStageBytes = size_t{8} << 20;  // one pinned staging buffer
constexpr int kReaders = 4;                       // reader threads, two buffers and one stream each
constexpr int kMaxDevices = 64;

struct Reader {
    hipStream_t stream = nullptr;
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};  // last copy out of buf[b] finished
};

struct StagePool {
    bool ready = false;
    Reader readers[kReaders];
};

std::mutex g_pool_mutex;  // one transfer at a time: the pool's buffers are shared
StagePool g_pools[kMaxDevices];

void pool_release(StagePool& p) {
    for (Reader& r : p.readers) {
        for (int b = 0; b < 2; ++b) {
            if (r.done[b] != nullptr) hipEventDestroy(r.done[b]);
            if (r.buf[b] != nullptr) hipHostFree(r.buf[b]);
            r.done[b] = nullptr;
            r.buf[b] = nullptr;
        }
        if (r.stream != nullptr) hipStreamDestroy(r.stream);
        r.stream = nullptr;
    }
    p.ready = false;
}

// Pinned buffers, streams (default priority) and events, made once per device
// and kept until the process ends.
int pool_for(int dev, StagePool** out) {
    StagePool& p = g_pools[dev];
    if (!p.ready) {
        hipError_t err = hipSuccess;
        for (Reader& r : p.readers) {
            if (err == hipSuccess) err = hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking);
            for (int b = 0; b < 2 && err == hipSuccess; ++b) {
                err = hipHostMalloc(&r.buf[b], kStageBytes, hipHostMallocDefault);
                if (err == hipSuccess) err = hipEventCreateWithFlags(&r.done[b], hipEventDisableTiming);
            }
        }
        if (err != hipSuccess) {
            pool_release(p);
            return plm::hip_fail(err, "file staging buffers");
        }
        p.ready = true;
    }
    *out = &p;
    return 0;
}

struct Chunk {
    uint64_t off;
    uint64_t len;
    char* dst;
};

// Read exactly len bytes at off.  0, or -errno / -EIO on a short file.
int read_full(int fd, void* buf, uint64_t len, uint64_t off) {
    char* p = static_cast<char*>(buf);
    while (len > 0) {
        const ssize_t n = pread(fd, p, static_cast<size_t>(len), static_cast<off_t>(off));
        if (n < 0) {
            if (errno == EINTR) continue;
            return -errno;
        }
        if (n == 0) return -EIO;
        p += n;
        len -= static_cast<uint64_t>(n);
        off += static_cast<uint64_t>(n);
    }
    return 0;
}

// One reader thread: chunks first, first + step, ... through its two buffers.
void reader_loop(int dev, int fd, Reader* r, const std::vector<Chunk>* chunks, size_t first, size_t step,
                 std::atomic<int>* status) {
    hipError_t err = hipSetDevice(dev);
    size_t k = 0;
    for (size_t i = first; i < chunks->size() && err == hipSuccess && status->load() == 0; i += step, ++k) {
        const Chunk& c = (*chunks)[i];
        const int b = static_cast<int>(k & 1);
        err = hipEventSynchronize(r->done[b]);  // the buffer's previous copy has left it
        if (err != hipSuccess) break;
        const int rc = read_full(fd, r->buf[b], c.len, c.off);
        if (rc != 0) {
            int expected = 0;
            status->compare_exchange_strong(expected, -5);
            break;
        }
        err = hipMemcpyAsync(c.dst, r->buf[b], c.len, hipMemcpyHostToDevice, r->stream);
        if (err == hipSuccess) err = hipEventRecord(r->done[b], r->stream);
    }
    const hipError_t sync = hipStreamSynchronize(r->stream);
    if (err == hipSuccess) err = sync;
    if (err != hipSuccess) {
        int expected = 0;
        status->compare_exchange_strong(expected, -(1000 + static_cast<int>(err)));
    }
}

// Byte ranges [off, off + len) of the file at path into device memory at dst
// (current device).  Returns when the bytes are in device memory.
int spans_to_device(const char* path, const uint64_t* offs, const uint64_t* lens, char* const* dsts, int64_t count) {
    if (path == nullptr || offs == nullptr || lens == nullptr || dsts == nullptr) return plm::fail(-1, "null pointer");
    if (count < 0) return plm::fail(-2, "negative span count");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return plm::fail(-5, "cannot open %s: %s", path, std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return plm::fail(-5, "cannot stat %s", path);
    }
    const uint64_t size = static_cast<uint64_t>(st.st_size);
    std::vector<Chunk> chunks;
    for (int64_t i = 0; i < count; ++i) {
        if (lens[i] == 0) continue;
        if (dsts[i] == nullptr || offs[i] > size || lens[i] > size - offs[i]) {
            close(fd);
            return plm::fail(-2, "span %lld lies outside %s or has no destination", static_cast<long long>(i), path);
        }
        for (uint64_t done = 0; done < lens[i]; done += kStageBytes) {
            const uint64_t n = lens[i] - done < kStageBytes ? lens[i] - done : kStageBytes;
            chunks.push_back(Chunk{offs[i] + done, n, dsts[i] + done});
        }
    }
    if (chunks.empty()) {
        close(fd);
        return 0;
    }
    posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);

    std::lock_guard<std::mutex> lock(g_pool_mutex);
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        close(fd);
        return err != hipSuccess ? plm::hip_fail(err, "hipGetDevice") : plm::fail(-2, "device index");
    }
    StagePool* pool = nullptr;
    int code = pool_for(dev, &pool);
    if (code != 0) {
        close(fd);
        return code;
    }
    // The destinations may have been handed out in the order of the caller's
    // stream: the readers' copies start after the work queued there.
    hipEvent_t ready = nullptr;
    err = hipEventCreateWithFlags(&ready, hipEventDisableTiming);
    if (err == hipSuccess) err = hipEventRecord(ready, plm::current_stream());
    for (int r = 0; r < kReaders && err == hipSuccess; ++r) err = hipStreamWaitEvent(pool->readers[r].stream, ready, 0);
    if (ready != nullptr) hipEventDestroy(ready);
    if (err != hipSuccess) {
        close(fd);
        return plm::hip_fail(err, "file transfer ordering");
    }

    const size_t nthreads = chunks.size() < static_cast<size_t>(kReaders) ? chunks.size() : kReaders;
    std::atomic<int> status{0};
    std::vector<std::thread> threads;
    for (size_t t = 0; t < nthreads; ++t)
        threads.emplace_back(reader_loop, dev, fd, &pool->readers[t], &chunks, t, nthreads, &status);
    for (std::thread& t : threads) t.join();
    close(fd);
    code = status.load();
    if (code == -5) return plm::fail(-5, "read of %s failed", path);
    if (code != 0) return plm::fail(code, "copy of %s to the device failed", path);
    return 0;
}

struct Row8DeviceTensor {
    void* data;
    uint64_t nbytes;
};

struct Row8MappedFile {
    int fd;
    uint8_t* base;
    uint64_t nbytes;
};

}  // namespace

// ====================================================================== C ABI

PLM_EXPORT int pocketlm_file_spans_to_device(const char* path, const uint64_t* file_offsets,
                                             const uint64_t* byte_lengths, const uint64_t* device_dsts,
                                             int64_t count) {
    plm::clear_error();
    std::vector<char*> dsts(static_cast<size_t>(count > 0 ? count : 0));
    if (device_dsts != nullptr)
        for (int64_t i = 0; i < count; ++i) dsts[i] = reinterpret_cast<char*>(static_cast<uintptr_t>(device_dsts[i]));
    return spans_to_device(path, file_offsets, byte_lengths, device_dsts != nullptr ? dsts.data() : nullptr, count);
}

PLM_EXPORT void* row8_artifact_load_tensor(const char* path, uint64_t offset, uint64_t nbytes) {
    plm::clear_error();
    if (path == nullptr || nbytes == 0 || (nbytes % 2) != 0) return nullptr;
    void* data = nullptr;
    if (hipMalloc(&data, nbytes) != hipSuccess) return nullptr;
    char* dst = static_cast<char*>(data);
    if (spans_to_device(path, &offset, &nbytes, &dst, 1) != 0) {
        hipFree(data);
        return nullptr;
    }
    return new Row8DeviceTensor{data, nbytes};
}

PLM_EXPORT void row8_artifact_free_tensor(void* handle) {
    Row8DeviceTensor* t = static_cast<Row8DeviceTensor*>(handle);
    if (t == nullptr) return;
    if (t->data != nullptr) hipFree(t->data);
    delete t;
}

PLM_EXPORT const uint16_t* row8_artifact_tensor_data(void* handle) {
    const Row8DeviceTensor* t = static_cast<const Row8DeviceTensor*>(handle);
    return t == nullptr ? nullptr : static_cast<const uint16_t*>(t->data);
}

PLM_EXPORT uint64_t row8_artifact_tensor_nbytes(void* handle) {
    const Row8DeviceTensor* t = static_cast<const Row8DeviceTensor*>(handle);
    return t == nullptr ? 0 : t->nbytes;
}

PLM_EXPORT void* row8_artifact_map_file(const char* path) {
    if (path == nullptr) return nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return nullptr;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return nullptr;
    }
    void* base = mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_SHARED, fd, 0);
    if (base == MAP_FAILED) {
        close(fd);
        return nullptr;
    }
    return new Row8MappedFile{fd, static_cast<uint8_t*>(base), static_cast<uint64_t>(st.st_size)};
}

PLM_EXPORT void row8_artifact_unmap_file(void* handle) {
    Row8MappedFile* m = static_cast<Row8MappedFile*>(handle);
    if (m == nullptr) return;
    if (m->base != nullptr) munmap(m->base, static_cast<size_t>(m->nbytes));
    if (m->fd >= 0) close(m->fd);
    delete m;
}

PLM_EXPORT const uint16_t* row8_artifact_mapped_data(void* handle, uint64_t offset, uint64_t nbytes) {
    const Row8MappedFile* m = static_cast<const Row8MappedFile*>(handle);
    if (m == nullptr || m->base == nullptr || (offset % 2) != 0 || (nbytes % 2) != 0) return nullptr;
    if (offset > m->nbytes || nbytes > m->nbytes - offset) return nullptr;
    return reinterpret_cast<const uint16_t*>(m->base + offset);
}

PLM_EXPORT uint64_t row8_artifact_mapped_nbytes(void* handle) {
    const Row8MappedFile* m = static_cast<const Row8MappedFile*>(handle);
    return m == nullptr ? 0 : m->nbytes;
}
