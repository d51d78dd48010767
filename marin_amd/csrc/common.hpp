// Internal host-side plumbing for libmarin_hip: errors, the device context, buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "marin_hip.h"

namespace marin {

// A failure carrying the marin_status and the fields of the matching reference error variant
// (crates/cuda/src/error.rs:6-36).
struct Error : std::runtime_error {
    marin_status status;
    size_t expected = 0, actual = 0, extra = 0;
    bool oom = false;
    Error(marin_status s, const std::string &msg, size_t e = 0, size_t a = 0, size_t x = 0)
        : std::runtime_error(msg), status(s), expected(e), actual(a), extra(x) {}
};

[[noreturn]] inline void shape(const char *what, size_t expected, size_t actual) {
    throw Error(MARIN_SHAPE,
                std::string(what) + ": expected " + std::to_string(expected) + ", got " + std::to_string(actual),
                expected, actual);
}
[[noreturn]] inline void unsupported(const char *what, size_t max, size_t actual) {
    throw Error(MARIN_UNSUPPORTED,
                std::string(what) + " must be between 1 and " + std::to_string(max) + ", got " +
                    std::to_string(actual),
                max, actual);
}
[[noreturn]] inline void overflow(const char *what) {
    throw Error(MARIN_OVERFLOW, std::string(what) + ": size arithmetic overflowed");
}
inline void check_len(const char *what, size_t expected, size_t actual) {
    if (expected != actual) shape(what, expected, actual);
}
inline size_t mul(size_t a, size_t b, const char *what) {
    size_t r;
    if (__builtin_mul_overflow(a, b, &r)) overflow(what);
    return r;
}
inline uint32_t to_u32(size_t v, const char *what) {
    if (v > 0xffffffffull) overflow(what);
    return (uint32_t)v;
}

inline void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        Error err(MARIN_DRIVER, std::string("HIP error in ") + what + ": " + hipGetErrorString(e));
        err.oom = e == hipErrorOutOfMemory;
        throw err;
    }
}
#define HIP_CHECK(call) ::marin::hip_check((call), #call)

// Error-to-status translation for every exported function.
void set_error(const Error &e);
void set_error(marin_status s, const std::string &msg);
void clear_error();

template <class F>
marin_status guard(F &&f) {
    try {
        f();
        return MARIN_OK;
    } catch (const Error &e) {
        set_error(e);
        return e.status;
    } catch (const std::bad_alloc &) {
        set_error(MARIN_DRIVER, "host allocation failed");
        return MARIN_DRIVER;
    } catch (const std::exception &e) {
        set_error(MARIN_DRIVER, e.what());
        return MARIN_DRIVER;
    }
}

size_t dtype_bytes(marin_dtype d);

// Instantiated HIP graphs still alive at process exit are destroyed by an atexit handler that runs before the HIP
// runtime's own teardown.
void register_graph(hipGraphExec_t g);
void unregister_graph(hipGraphExec_t g);

}  // namespace marin

// Device memory with the context that owns it.
struct marin_buffer {
    marin_gpu *gpu = nullptr;
    void *data = nullptr;
    size_t len = 0;  // elements
    marin_dtype dtype = MARIN_F32;
    size_t bytes() const { return len * marin::dtype_bytes(dtype); }
};

struct marin_tokens {
    marin_gpu *gpu = nullptr;
    uint32_t *data = nullptr;
    size_t capacity = 0;
};

struct marin_gpu {
    int device = 0;
    hipStream_t stream = nullptr;
    int cu_count = 0;
    std::string name, arch;
    // Counters of crates/cuda/src/counters.rs:10-89.
    marin_traffic traffic{};
    // Pinned staging for small host->device copies (token ids, page addresses).
    void *pinned = nullptr;
    size_t pinned_bytes = 0;

    // Every device allocation made through alloc() holds the context: marin_gpu_free only marks it closing, and the
    // context is destroyed when its last allocation is released (as the reference's buffers hold an Arc of their
    // context), so objects may be freed in any order.
    size_t live = 0;
    bool closing = false;
    void *alloc(size_t bytes, bool zero = true);
    void release(void *p);
    void destroy();
    void upload(void *dst, const void *src, size_t bytes);  // synchronous with respect to the host data
    void download(void *dst, const void *src, size_t bytes);
    void *stage(const void *src, size_t bytes);  // copies into pinned memory; valid until the next stage()
    // Grow-only device scratch for multi-token products (activation limbs); waits for the stream before it grows.
    // Never reached by a one-token decode step.
    void *work = nullptr;
    size_t work_bytes = 0;
    void *workspace(size_t bytes);
    // While set, workspace() hands out this caller-owned device memory instead (and refuses a larger request with
    // Unsupported), so a call allocates nothing (the allocation-free entry points).
    void *fixed_work = nullptr;
    size_t fixed_work_bytes = 0;
    // Device fault word: kernels that meet input the reference rejects (non-finite router logits) set a bit and
    // carry on with harmless values; the next blocking call (synchronize, download) reports it and clears it.
    uint32_t *fault = nullptr;
    void check_fault();
    // 4 KiB of zeros on the device: the row the one-token attention reads for positions past a context.
    void *zero_row = nullptr;
    // Gpu::set_fast_attention (crates/cuda/src/attention.rs:81-86): prompt passes over an f16 cache use the
    // matrix-core attention when set (the default; MARIN_NO_FA=1 in the environment clears it at creation).
    bool fast_attention = true;

    // Launch accounting. With a profile attached, every launch is tagged with its kind, algorithmic bytes and kernel
    // name. The product and attention launchers then launch through hipExtLaunchKernelGGL with the two events of
    // kernel_events(), which the runtime records at that kernel's own start and end; any other launch records one
    // event after itself and runs from the previous event.
    enum Kind { OTHER = 0, GEMV = 1, ATTENTION = 2 };
    struct ProfileEntry {
        hipEvent_t start;  // nullptr: from the previous entry's event
        hipEvent_t event;
        int kind;
        double bytes;
        const char *name;
    };
    std::vector<ProfileEntry> *profile = nullptr;
    std::vector<hipEvent_t> event_pool;
    size_t events_used = 0;
    hipEvent_t pending_start = nullptr, pending_stop = nullptr;
    // When set, product and attention launchers skip every kernel whose name differs (single-kernel timing graphs);
    // a launcher that skipped sets `skipped` so no launch is counted.
    const char *only = nullptr;
    bool skipped = false;
    hipEvent_t next_event();
    // Two events for a kernel's own start and end when profiling (both nullptr otherwise); launched() takes them.
    void kernel_events(hipEvent_t &start, hipEvent_t &stop);
    void launched(int kind = OTHER, double bytes = 0.0, const char *name = nullptr);
};

namespace marin {
// Bits of marin_gpu::fault.
constexpr uint32_t FAULT_ROUTER_NONFINITE = 1u;
}  // namespace marin
