// Operand binding for one library call.
//
// Device operands are used in place. Host operands are staged through the
// device pool: inputs are copied in on the SDK stream before the kernel
// (through pinned chunks, so the caller's memory has been read when bind
// returns), outputs are copied back after it, and finish() returns once the
// host memory is written. Any HIP failure is recorded once and reported by
// finish().
#pragma once

#include "pinned.hpp"
#include "sdk.hpp"

#include <stddef.h>

namespace icsdk {

class Staging {
public:
    Staging(const char *op, bool host, char *error, size_t capacity)
        : op_(op), host_(host), error_(error), capacity_(capacity) {}
    Staging(const Staging &) = delete;
    Staging &operator=(const Staging &) = delete;
    ~Staging() {
        // an abandoned host call may still have kernels in flight on its
        // staging blocks; later users of the blocks enqueue after them on the
        // same stream, but drain anyway so a failed call leaves nothing behind
        if (host_ && count_ > 0 && !synced_) (void)hipStreamSynchronize(stream_);
        for (int i = 0; i < count_; ++i) scratch_release(slots_[i].device, slots_[i].pooled);
    }

    // Must be called (and succeed) before binding operands.
    bool begin() {
        if (!sdk_ready(error_, capacity_)) return false;
        stream_ = sdk_stream();
        return true;
    }
    hipStream_t stream() const { return stream_; }
    bool host() const { return host_; }

    // Host-data pointers (or device addresses when !host) of `bytes` bytes.
    const void *in(const void *data, size_t bytes) { return bind(const_cast<void *>(data), bytes, true, false); }
    void *out(void *data, size_t bytes) { return bind(data, bytes, false, true); }
    void *inout(void *data, size_t bytes) { return bind(data, bytes, true, true); }

    // Checks the launch status, copies host outputs back and waits.
    bool finish(hipError_t launch_status) {
        if (failed_) return false;
        if (launch_status != hipSuccess) {
            set_error(error_, capacity_, "%s: kernel launch failed: %s", op_,
                      hipGetErrorString(launch_status));
            return false;
        }
        if (host_) {
            bool copied = false;
            for (int i = 0; i < count_; ++i) {
                if (!slots_[i].copy_out || slots_[i].bytes == 0) continue;
                if (!pinned_to_host(slots_[i].host, slots_[i].device, slots_[i].bytes, stream_,
                                    error_, capacity_)) {
                    failed_ = true;
                    return false;
                }
                copied = true;
            }
            // each output copy waited for the work before it; with none, wait here
            synced_ = copied || check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
            return synced_;
        }
        return true;
    }

    bool failed() const { return failed_; }

private:
    struct Slot {
        void *host;
        void *device;
        size_t bytes;   // caller bytes to copy
        size_t pooled;  // size of the staging block
        bool copy_out;
    };

    void *bind(void *data, size_t bytes, bool copy_in, bool copy_out) {
        if (!host_ || data == nullptr || failed_) return data;
        if (count_ == kMaxSlots) {
            failed_ = true;
            set_error(error_, capacity_, "%s: too many staged operands", op_);
            return nullptr;
        }
        const size_t size = bytes == 0 ? 1 : bytes;
        void *device = scratch_acquire(size);
        if (device == nullptr) {
            failed_ = true;
            set_error(error_, capacity_, "%s: out of device memory staging %zu bytes", op_, bytes);
            return nullptr;
        }
        slots_[count_++] = Slot{data, device, bytes, size, copy_out};
        if (copy_in && bytes > 0 &&
            !pinned_to_device(device, data, bytes, stream_, error_, capacity_)) {
            failed_ = true;
            return nullptr;
        }
        return device;
    }

    bool check(hipError_t status, const char *what) {
        if (status == hipSuccess) return true;
        if (!failed_) set_error(error_, capacity_, "%s: %s failed: %s", op_, what,
                                hipGetErrorString(status));
        failed_ = true;
        return false;
    }

    static constexpr int kMaxSlots = 8;
    const char *op_;
    bool host_;
    char *error_;
    size_t capacity_;
    hipStream_t stream_ = nullptr;
    Slot slots_[kMaxSlots] = {};
    int count_ = 0;
    bool failed_ = false;
    bool synced_ = false;
};

}  // namespace icsdk
