// Device context, buffers, events and error reporting of the C ABI (crates/cuda/src/gpu.rs, counters.rs, error.rs).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <set>

#include "common.hpp"
#include "ops.hpp"

namespace marin {

struct LastError {
    std::string msg;
    size_t expected = 0, actual = 0, extra = 0;
    bool oom = false;
};
static thread_local LastError g_last;

void set_error(const Error &e) {
    g_last.msg = e.what();
    g_last.expected = e.expected;
    g_last.actual = e.actual;
    g_last.extra = e.extra;
    g_last.oom = e.oom;
}
void set_error(marin_status, const std::string &msg) {
    g_last = LastError{};
    g_last.msg = msg;
}
void clear_error() { g_last = LastError{}; }

size_t dtype_bytes(marin_dtype d) {
    switch (d) {
        case MARIN_F32:
        case MARIN_U32: return 4;
        case MARIN_BF16:
        case MARIN_F16: return 2;
        case MARIN_U8: return 1;
    }
    return 4;
}

static std::mutex g_graph_mutex;
static std::set<hipGraphExec_t> *g_graphs = nullptr;

void register_graph(hipGraphExec_t g) {
    std::lock_guard<std::mutex> lock(g_graph_mutex);
    if (!g_graphs) g_graphs = new std::set<hipGraphExec_t>();
    g_graphs->insert(g);
}

void unregister_graph(hipGraphExec_t g) {
    std::lock_guard<std::mutex> lock(g_graph_mutex);
    if (g_graphs) g_graphs->erase(g);
}

static void destroy_graphs_at_exit() {
    std::lock_guard<std::mutex> lock(g_graph_mutex);
    if (!g_graphs) return;
    (void)hipDeviceSynchronize();
    for (hipGraphExec_t g : *g_graphs) (void)hipGraphExecDestroy(g);
    g_graphs->clear();
}

}  // namespace marin

using namespace marin;

void *marin_gpu::alloc(size_t bytes, bool zero) {
    void *p = nullptr;
    if (bytes == 0) bytes = 4;
    hipError_t e = hipMalloc(&p, bytes);
    hip_check(e, "hipMalloc");
    traffic.allocations++;
    live++;
    if (zero) {
        HIP_CHECK(hipMemsetAsync(p, 0, bytes, stream));
    }
    return p;
}

void marin_gpu::release(void *p) {
    if (!p) return;
    (void)hipFree(p);
    live--;
    if (closing && live == 0) destroy();
}

void *marin_gpu::workspace(size_t bytes) {
    if (fixed_work) {
        if (bytes > fixed_work_bytes) unsupported("scratch bytes of an allocation-free call", fixed_work_bytes, bytes);
        return fixed_work;
    }
    if (bytes <= work_bytes) return work;
    HIP_CHECK(hipStreamSynchronize(stream));
    if (work) (void)hipFree(work);
    work = nullptr;
    work_bytes = 0;
    const size_t want = std::max<size_t>(bytes, (size_t)1 << 22);
    hip_check(hipMalloc(&work, want), "hipMalloc (workspace)");
    work_bytes = want;
    traffic.allocations++;
    return work;
}

void marin_gpu::destroy() {
    (void)hipStreamSynchronize(stream);
    if (work) (void)hipFree(work);
    if (fault) (void)hipFree(fault);
    if (zero_row) (void)hipFree(zero_row);
    if (pinned) (void)hipHostFree(pinned);
    for (hipEvent_t e : event_pool) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(stream);
    delete this;
}

void marin_gpu::upload(void *dst, const void *src, size_t bytes) {
    if (!bytes) return;
    // Pageable host memory: a blocking copy ordered after the stream's earlier work.
    HIP_CHECK(hipStreamSynchronize(stream));
    HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    traffic.uploads++;
    traffic.upload_bytes += bytes;
}

void marin_gpu::download(void *dst, const void *src, size_t bytes) {
    if (!bytes) return;
    HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream));
    HIP_CHECK(hipStreamSynchronize(stream));
    traffic.downloads++;
    traffic.download_bytes += bytes;
    check_fault();
}

void marin_gpu::check_fault() {
    if (!fault) return;
    uint32_t word = 0;
    HIP_CHECK(hipMemcpy(&word, fault, 4, hipMemcpyDeviceToHost));
    if (!word) return;
    HIP_CHECK(hipMemset(fault, 0, 4));
    if (word & FAULT_ROUTER_NONFINITE)
        // ModelError::InvalidConfig("nonfinite ... router logits"), model/src/granite/layer.rs:42-47
        throw Error(MARIN_SELF_CHECK, "nonfinite router logits (their tokens were routed to experts 0..k-1 with "
                                      "weight 0)");
    throw Error(MARIN_SELF_CHECK, "device fault word " + std::to_string(word));
}

hipEvent_t marin_gpu::next_event() {
    if (events_used >= event_pool.size()) {
        hipEvent_t e;
        HIP_CHECK(hipEventCreate(&e));
        event_pool.push_back(e);
    }
    return event_pool[events_used++];
}

void marin_gpu::kernel_events(hipEvent_t &start, hipEvent_t &stop) {
    start = stop = nullptr;
    if (!profile) return;
    start = pending_start = next_event();
    stop = pending_stop = next_event();
}

void marin_gpu::launched(int kind, double bytes, const char *name) {
    traffic.launches++;
    if (!profile) return;
    hipEvent_t e = pending_stop;
    if (!e) {
        e = next_event();
        HIP_CHECK(hipEventRecord(e, stream));
    }
    profile->push_back({pending_start, e, kind, bytes, name});
    pending_start = pending_stop = nullptr;
}

void *marin_gpu::stage(const void *src, size_t bytes) {
    if (bytes > pinned_bytes) {
        HIP_CHECK(hipStreamSynchronize(stream));
        if (pinned) (void)hipHostFree(pinned);
        pinned = nullptr;
        pinned_bytes = 0;
        size_t want = std::max<size_t>(bytes, 1 << 16);
        HIP_CHECK(hipHostMalloc(&pinned, want, hipHostMallocDefault));
        pinned_bytes = want;
    } else {
        // The previous staged copy must have left the pinned area before it is overwritten.
        HIP_CHECK(hipStreamSynchronize(stream));
    }
    std::memcpy(pinned, src, bytes);
    return pinned;
}

extern "C" {

const char *marin_last_error(void) { return g_last.msg.c_str(); }
void marin_last_error_fields(size_t *expected, size_t *actual, size_t *extra) {
    if (expected) *expected = g_last.expected;
    if (actual) *actual = g_last.actual;
    if (extra) *extra = g_last.extra;
}
int marin_last_error_is_oom(void) { return g_last.oom ? 1 : 0; }

marin_status marin_gpu_new(marin_gpu **out) {
    return guard([&] {
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
            throw Error(MARIN_UNAVAILABLE, "no HIP device is visible");
        hipDeviceProp_t prop;
        HIP_CHECK(hipGetDeviceProperties(&prop, 0));
        std::string arch = prop.gcnArchName;
        if (arch.rfind("gfx950", 0) != 0)
            throw Error(MARIN_UNAVAILABLE, "device 0 is " + arch + "; this library is built for gfx950 only");
        HIP_CHECK(hipSetDevice(0));
        // Registered after the runtime is up, so it runs before the runtime's exit handlers.
        static std::once_flag once;
        std::call_once(once, [] { std::atexit(destroy_graphs_at_exit); });
        auto *g = new marin_gpu();
        g->device = 0;
        g->cu_count = prop.multiProcessorCount;
        g->name = prop.name;
        if (g->name.empty()) {
            char nm[256] = {0};
            if (hipDeviceGetName(nm, sizeof(nm) - 1, 0) == hipSuccess) g->name = nm;
        }
        if (g->name.empty())
            g->name = "AMD " + arch.substr(0, arch.find(':')) + " (" + std::to_string(prop.multiProcessorCount) + " CUs)";
        g->arch = arch;
        {
            const char *nofa = getenv("MARIN_NO_FA");
            g->fast_attention = !(nofa && *nofa && *nofa != '0');
        }
        hipError_t e = hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking);
        if (e != hipSuccess) {
            delete g;
            hip_check(e, "hipStreamCreate");
        }
        e = hipMalloc((void **)&g->fault, 256);
        if (e == hipSuccess) e = hipMemset(g->fault, 0, 256);
        if (e == hipSuccess) e = hipMalloc(&g->zero_row, 4096);
        if (e == hipSuccess) e = hipMemset(g->zero_row, 0, 4096);
        if (e != hipSuccess) {
            (void)hipStreamDestroy(g->stream);
            if (g->fault) (void)hipFree(g->fault);
            if (g->zero_row) (void)hipFree(g->zero_row);
            delete g;
            hip_check(e, "hipMalloc (fault word)");
        }
        *out = g;
    });
}

void marin_gpu_free(marin_gpu *g) {
    if (!g || g->closing) return;
    (void)hipStreamSynchronize(g->stream);
    forget_rope_frequencies(g);
    g->closing = true;
    if (g->live == 0) g->destroy();
}

marin_status marin_gpu_info_get(marin_gpu *g, marin_gpu_info *out) {
    return guard([&] {
        std::memset(out, 0, sizeof(*out));
        std::snprintf(out->name, sizeof(out->name), "%s", g->name.c_str());
        std::snprintf(out->arch, sizeof(out->arch), "%s", g->arch.c_str());
        out->compute_units = g->cu_count;
        HIP_CHECK(hipMemGetInfo(&out->free_bytes, &out->total_bytes));
    });
}

marin_status marin_gpu_synchronize(marin_gpu *g) {
    return guard([&] {
        HIP_CHECK(hipStreamSynchronize(g->stream));
        g->check_fault();
    });
}

void *marin_gpu_stream(marin_gpu *g) { return (void *)g->stream; }

marin_status marin_gpu_bind_to_thread(marin_gpu *g) {
    return guard([&] { HIP_CHECK(hipSetDevice(g->device)); });
}

void marin_set_fast_attention(marin_gpu *g, int on) { g->fast_attention = on != 0; }

marin_status marin_gpu_traffic(marin_gpu *g, marin_traffic *out) {
    return guard([&] { *out = g->traffic; });
}

struct marin_mark {
    hipEvent_t event;
};

marin_status marin_mark_new(marin_gpu *g, marin_mark **out) {
    return guard([&] {
        auto *m = new marin_mark();
        hipError_t e = hipEventCreate(&m->event);
        if (e != hipSuccess) {
            delete m;
            hip_check(e, "hipEventCreate");
        }
        HIP_CHECK(hipEventRecord(m->event, g->stream));
        *out = m;
    });
}

marin_status marin_mark_since(marin_mark *later, marin_mark *earlier, double *seconds) {
    return guard([&] {
        HIP_CHECK(hipEventSynchronize(later->event));
        float ms = 0;
        HIP_CHECK(hipEventElapsedTime(&ms, earlier->event, later->event));
        *seconds = ms * 1e-3;
    });
}

void marin_mark_free(marin_mark *m) {
    if (!m) return;
    (void)hipEventDestroy(m->event);
    delete m;
}

static marin_buffer *new_buffer(marin_gpu *g, marin_dtype dtype, size_t len) {
    auto *b = new marin_buffer();
    b->gpu = g;
    b->dtype = dtype;
    b->len = len;
    try {
        b->data = g->alloc(b->bytes(), true);
    } catch (...) {
        delete b;
        throw;
    }
    return b;
}

marin_status marin_buffer_zeros(marin_gpu *g, size_t len, marin_buffer **out) {
    return guard([&] {
        mul(len, 4, "buffer");
        *out = new_buffer(g, MARIN_F32, len);
    });
}

marin_status marin_buffer_upload(marin_gpu *g, const float *values, size_t len, marin_buffer **out) {
    return guard([&] {
        mul(len, 4, "buffer");
        marin_buffer *b = new_buffer(g, MARIN_F32, len);
        try {
            g->upload(b->data, values, len * 4);
        } catch (...) {
            g->release(b->data);
            delete b;
            throw;
        }
        *out = b;
    });
}

marin_status marin_buffer_upload_into(marin_gpu *g, const float *values, size_t len, marin_buffer *dst) {
    return guard([&] {
        check_len("upload length", dst->len, len);
        g->upload(dst->data, values, len * 4);
    });
}

marin_status marin_buffer_download(marin_gpu *g, const marin_buffer *b, float *dst, size_t len) {
    return guard([&] {
        if (b->dtype != MARIN_F32) shape("buffer element size", 4, dtype_bytes(b->dtype));
        check_len("download length", b->len, len);
        g->download(dst, b->data, len * 4);
    });
}

marin_status marin_buffer_download_range(marin_gpu *g, const marin_buffer *b, size_t start, size_t len, float *dst) {
    return guard([&] {
        if (start > b->len || len > b->len - start) shape("download range", b->len, start + len);
        g->download(dst, (const float *)b->data + start, len * 4);
    });
}

marin_status marin_buffer_copy_range_into(marin_gpu *g, const marin_buffer *src, size_t start, marin_buffer *dst) {
    return guard([&] {
        if (start > src->len || dst->len > src->len - start) shape("copy range", src->len, start + dst->len);
        if (!dst->len) return;
        HIP_CHECK(hipMemcpyAsync(dst->data, (const float *)src->data + start, dst->len * 4,
                                 hipMemcpyDeviceToDevice, g->stream));
    });
}

marin_status marin_buffer_copy_into_range(marin_gpu *g, const marin_buffer *src, marin_buffer *dst, size_t start) {
    return guard([&] {
        if (start > dst->len || src->len > dst->len - start) shape("copy range", dst->len, start + src->len);
        if (!src->len) return;
        HIP_CHECK(hipMemcpyAsync((float *)dst->data + start, src->data, src->len * 4, hipMemcpyDeviceToDevice,
                                 g->stream));
    });
}

size_t marin_buffer_len(const marin_buffer *b) { return b->len; }
marin_dtype marin_buffer_dtype(const marin_buffer *b) { return b->dtype; }
void *marin_buffer_device_ptr(const marin_buffer *b) { return b->data; }

void marin_buffer_free(marin_buffer *b) {
    if (!b) return;
    (void)hipStreamSynchronize(b->gpu->stream);
    b->gpu->release(b->data);
    delete b;
}

marin_status marin_buffer_new_typed(marin_gpu *g, marin_dtype dtype, size_t len, const void *host,
                                    marin_buffer **out) {
    return guard([&] {
        mul(len, dtype_bytes(dtype), "buffer");
        marin_buffer *b = new_buffer(g, dtype, len);
        if (host) {
            try {
                g->upload(b->data, host, b->bytes());
            } catch (...) {
                g->release(b->data);
                delete b;
                throw;
            }
        }
        *out = b;
    });
}

marin_status marin_buffer_download_raw(marin_gpu *g, const marin_buffer *b, void *dst, size_t bytes) {
    return guard([&] {
        check_len("download bytes", b->bytes(), bytes);
        g->download(dst, b->data, bytes);
    });
}

marin_status marin_tokens_new(marin_gpu *g, size_t capacity, marin_tokens **out) {
    return guard([&] {
        auto *t = new marin_tokens();
        t->gpu = g;
        t->capacity = capacity;
        try {
            t->data = (uint32_t *)g->alloc(mul(std::max<size_t>(capacity, 1), 4, "tokens"), true);
        } catch (...) {
            delete t;
            throw;
        }
        *out = t;
    });
}

void marin_tokens_free(marin_tokens *t) {
    if (!t) return;
    (void)hipStreamSynchronize(t->gpu->stream);
    t->gpu->release(t->data);
    delete t;
}

}  // extern "C"
