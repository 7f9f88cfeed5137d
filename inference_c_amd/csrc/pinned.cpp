// Pinned staging: a pool of page-locked host chunks (hipHostMalloc, never
// hipHostRegister) with one completion event each, and a few persistent
// worker threads for large host copies.
//
// A transfer takes all the chunks it will use at once (at most kPerCall), so
// no thread ever holds chunks while waiting for more. Host-to-device: copy
// piece i into chunk i % n (after that chunk's previous DMA has finished),
// enqueue its DMA, record the chunk's event. Device-to-host: enqueue the
// DMAs of the first n pieces, then for each piece wait for its event, copy
// it out and enqueue the DMA of piece i + n into the freed chunk.
#include "pinned.hpp"

#include "sdk.hpp"

#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace icsdk {
namespace {

constexpr size_t kChunkBytes = 4u << 20;
constexpr int kMaxChunks = 16;
constexpr int kPerCall = 3;
constexpr size_t kParallelBytes = 1u << 20;  // host copies from here on use the workers
constexpr int kWorkers = 3;                  // plus the calling thread

struct Chunk {
    char *host = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;  // an event has been recorded since the last wait
};

class ChunkPool {
public:
    bool acquire(int n, Chunk **out, char *error, size_t capacity) {
        std::unique_lock<std::mutex> lock(mutex_);
        while ((int)free_.size() < n && total_ + (n - (int)free_.size()) > kMaxChunks)
            cv_.wait(lock);
        while ((int)free_.size() < n) {
            Chunk *c = new Chunk;
            if (hipHostMalloc(reinterpret_cast<void **>(&c->host), kChunkBytes,
                              hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&c->done, hipEventDisableTiming) != hipSuccess) {
                if (c->host) (void)hipHostFree(c->host);
                delete c;
                set_error(error, capacity, "pinned staging: cannot allocate page-locked memory");
                return false;
            }
            free_.push_back(c);
            ++total_;
        }
        for (int i = 0; i < n; ++i) {
            out[i] = free_.back();
            free_.pop_back();
        }
        return true;
    }

    void release(int n, Chunk **chunks) {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            for (int i = 0; i < n; ++i) free_.push_back(chunks[i]);
        }
        cv_.notify_all();
    }

    void trim() {
        std::vector<Chunk *> idle;
        {
            std::lock_guard<std::mutex> lock(mutex_);
            idle.swap(free_);
            total_ -= (int)idle.size();
        }
        for (Chunk *c : idle) {
            if (c->pending) (void)hipEventSynchronize(c->done);
            (void)hipEventDestroy(c->done);
            (void)hipHostFree(c->host);
            delete c;
        }
        cv_.notify_all();
    }

private:
    std::mutex mutex_;
    std::condition_variable cv_;
    std::vector<Chunk *> free_;
    int total_ = 0;
};

ChunkPool &chunk_pool() {
    static ChunkPool *pool = new ChunkPool;  // outlives static destructors
    return *pool;
}

// memcpy split over kWorkers persistent threads and the caller. One large
// copy runs at a time; a caller that finds the workers busy copies alone.
class CopyWorkers {
public:
    CopyWorkers() {
        for (int i = 0; i < kWorkers; ++i) std::thread([this, i] { run(i); }).detach();
    }

    void copy(char *dst, const char *src, size_t bytes) {
        std::unique_lock<std::mutex> busy(busy_, std::try_to_lock);
        if (bytes < kParallelBytes || !busy.owns_lock()) {
            std::memcpy(dst, src, bytes);
            return;
        }
        // ceil(bytes / (kWorkers + 1)) rounded up to 64: the parts cover every byte
        const size_t part = ((bytes + kWorkers) / (kWorkers + 1) + 63) & ~size_t(63);
        {
            std::lock_guard<std::mutex> lock(mutex_);
            for (int i = 0; i < kWorkers; ++i) {
                const size_t first = part * (i + 1);
                tasks_[i] = Task{dst + first, src + first,
                                 first >= bytes ? 0 : std::min(part, bytes - first)};
            }
            left_ = kWorkers;
            ++generation_;
        }
        start_.notify_all();
        std::memcpy(dst, src, std::min(part, bytes));
        std::unique_lock<std::mutex> lock(mutex_);
        done_.wait(lock, [this] { return left_ == 0; });
    }

private:
    struct Task {
        char *dst;
        const char *src;
        size_t bytes;
    };

    void run(int index) {
        uint64_t seen = 0;
        for (;;) {
            Task task;
            {
                std::unique_lock<std::mutex> lock(mutex_);
                start_.wait(lock, [&] { return generation_ != seen; });
                seen = generation_;
                task = tasks_[index];
            }
            if (task.bytes) std::memcpy(task.dst, task.src, task.bytes);
            std::lock_guard<std::mutex> lock(mutex_);
            if (--left_ == 0) done_.notify_all();
        }
    }

    std::mutex busy_;
    std::mutex mutex_;
    std::condition_variable start_, done_;
    Task tasks_[kWorkers] = {};
    int left_ = 0;
    uint64_t generation_ = 0;
};

CopyWorkers &copy_workers() {
    static CopyWorkers *workers = new CopyWorkers;  // threads are detached; never destroyed
    return *workers;
}

void host_copy(char *dst, const char *src, size_t bytes) {
    copy_workers().copy(dst, src, bytes);
}

int chunks_for(size_t bytes) {
    const size_t pieces = (bytes + kChunkBytes - 1) / kChunkBytes;
    return pieces < (size_t)kPerCall ? (int)pieces : kPerCall;
}

// Waits until the chunk's last DMA has finished.
bool settle(Chunk *c, char *error, size_t capacity) {
    if (!c->pending) return true;
    c->pending = false;
    return hip_ok(hipEventSynchronize(c->done), "pinned staging: hipEventSynchronize", error,
                  capacity);
}

bool record(Chunk *c, hipStream_t stream, char *error, size_t capacity) {
    c->pending = true;
    return hip_ok(hipEventRecord(c->done, stream), "pinned staging: hipEventRecord", error,
                  capacity);
}

}  // namespace

bool pinned_to_device(void *dst, const void *src, size_t bytes, hipStream_t stream,
                      char *error, size_t capacity) {
    if (bytes == 0) return true;
    Chunk *chunks[kPerCall];
    const int n = chunks_for(bytes);
    if (!chunk_pool().acquire(n, chunks, error, capacity)) return false;
    bool ok = true;
    size_t i = 0;
    for (size_t off = 0; ok && off < bytes; off += kChunkBytes, ++i) {
        Chunk *c = chunks[i % n];
        const size_t piece = std::min(kChunkBytes, bytes - off);
        ok = settle(c, error, capacity);
        if (!ok) break;
        host_copy(c->host, static_cast<const char *>(src) + off, piece);
        ok = hip_ok(hipMemcpyAsync(static_cast<char *>(dst) + off, c->host, piece,
                                   hipMemcpyHostToDevice, stream),
                    "pinned staging: host-to-device copy", error, capacity) &&
             record(c, stream, error, capacity);
    }
    chunk_pool().release(n, chunks);
    return ok;
}

bool pinned_to_host(void *dst, const void *src, size_t bytes, hipStream_t stream, char *error,
                    size_t capacity) {
    if (bytes == 0) return true;
    Chunk *chunks[kPerCall];
    const int n = chunks_for(bytes);
    if (!chunk_pool().acquire(n, chunks, error, capacity)) return false;
    const size_t pieces = (bytes + kChunkBytes - 1) / kChunkBytes;
    auto enqueue = [&](size_t i) {
        Chunk *c = chunks[i % n];
        const size_t off = i * kChunkBytes;
        return settle(c, error, capacity) &&
               hip_ok(hipMemcpyAsync(c->host, static_cast<const char *>(src) + off,
                                     std::min(kChunkBytes, bytes - off), hipMemcpyDeviceToHost,
                                     stream),
                      "pinned staging: device-to-host copy", error, capacity) &&
               record(c, stream, error, capacity);
    };
    bool ok = true;
    for (size_t i = 0; ok && i < pieces && i < (size_t)n; ++i) ok = enqueue(i);
    for (size_t i = 0; ok && i < pieces; ++i) {
        Chunk *c = chunks[i % n];
        const size_t off = i * kChunkBytes;
        ok = settle(c, error, capacity);
        if (!ok) break;
        host_copy(static_cast<char *>(dst) + off, c->host, std::min(kChunkBytes, bytes - off));
        if (i + n < pieces) ok = enqueue(i + n);
    }
    // a failed call leaves no DMA behind into a chunk that goes back to the pool
    for (int k = 0; k < n; ++k) (void)settle(chunks[k], nullptr, 0);
    chunk_pool().release(n, chunks);
    return ok;
}

void pinned_release() { chunk_pool().trim(); }

}  // namespace icsdk
