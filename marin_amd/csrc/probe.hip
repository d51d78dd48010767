// Bandwidth probe (the role of crates/cuda/src/probe.rs:145-314 and probe.cu:4-68 of the reference, which measure
// HBM read rate with their own kernels): a plain device-to-device copy of a known byte count. It calibrates the
// profiler's memory counters (FETCH_SIZE / WRITE_SIZE per dispatch against the bytes the copy must move) and gives
// the streaming rate the decode kernels are compared with.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "marin_hip.h"
#include "common.hpp"

namespace marin {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Each thread copies 16-byte words n = i, i + stride, ... (n16 words in all).
__global__ __launch_bounds__(256) void probe_copy(const u32x4 *__restrict__ src, u32x4 *__restrict__ dst, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace marin

using namespace marin;

extern "C" {

marin_status marin_probe_copy(marin_gpu *g, size_t bytes, int reps, double *seconds) {
    return guard([&] {
        if (bytes == 0 || bytes % 16) shape("probe copy bytes (a multiple of 16)", 16, bytes);
        if (reps < 1) shape("probe copy repetitions", 1, (size_t)reps);
        void *src = g->alloc(bytes, true);
        void *dst = nullptr;
        try {
            dst = g->alloc(bytes, false);
            const int blocks = std::max(g->cu_count, 1) * 8;
            hipEvent_t a, b;
            HIP_CHECK(hipEventCreate(&a));
            HIP_CHECK(hipEventCreate(&b));
            probe_copy<<<blocks, 256, 0, g->stream>>>((const u32x4 *)src, (u32x4 *)dst, bytes / 16);
            HIP_CHECK(hipEventRecord(a, g->stream));
            for (int r = 0; r < reps; ++r)
                probe_copy<<<blocks, 256, 0, g->stream>>>((const u32x4 *)src, (u32x4 *)dst, bytes / 16);
            HIP_CHECK(hipEventRecord(b, g->stream));
            HIP_CHECK(hipEventSynchronize(b));
            float ms = 0.0f;
            HIP_CHECK(hipEventElapsedTime(&ms, a, b));
            (void)hipEventDestroy(a);
            (void)hipEventDestroy(b);
            *seconds = ms * 1e-3 / reps;
        } catch (...) {
            g->release(src);
            if (dst) g->release(dst);
            throw;
        }
        g->release(src);
        g->release(dst);
    });
}

}  // extern "C"
