// The allocation-free quantized product: marin_matmul_quant_bf16 with its multi-token scratch (the activation limbs,
// exponents and per-token factors of the batch and prompt products) in a fixed device array of this library instead
// of memory it allocates, for callers that cannot allocate (code under HIP graph capture, serving loops, harnesses
// that forbid hipMalloc). No reference counterpart.
//
// The array is one per device for the life of the process. Every call on a device shares it and it keeps the last
// call's contents (the kernels write every byte they read, so nothing needs clearing); two calls that overlap on one
// device (two contexts' streams running at once) race on it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "gemm.hpp"
#include "gemv.hpp"

namespace marin {

constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)4 << 20;  // 4 MiB: 64 tokens of 12288 columns
constexpr int NOALLOC_MAX_DEVICES = 64;

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

// The device address of `scratch` on `device`, looked up once per device with that device current. Host code uses
// only this address, never the array's name (a host-side stand-in).
static void *scratch_on(int device) {
    static std::mutex mu;
    static void *ptrs[NOALLOC_MAX_DEVICES] = {};
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) unsupported("device index", NOALLOC_MAX_DEVICES - 1, (size_t)device);
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[device]) {
        int current = 0;
        HIP_CHECK(hipGetDevice(&current));
        if (current != device) HIP_CHECK(hipSetDevice(device));
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (current != device) (void)hipSetDevice(current);
        hip_check(e, "hipGetSymbolAddress (allocation-free scratch)");
        if (!p) throw Error(MARIN_DRIVER, "the allocation-free scratch has no device address");
        ptrs[device] = p;
    }
    return ptrs[device];
}

// Scratch a product of `tokens` rows over w's columns may ask for: the limb layout of the batch product (tokens
// padded to whole tiles of 4), which also bounds the prompt product's.
static size_t product_scratch_bound(const marin_quant_matrix *w, size_t tokens) {
    if (tokens <= 1) return 0;
    return moe_gate_up_workspace((tokens + 3) / 4 * 4, w->cols, w->group) + 256;
}

}  // namespace marin

using namespace marin;

extern "C" marin_status marin_matmul_quant_bf16_noalloc(marin_gpu *g, const marin_quant_matrix *w,
                                                        const marin_buffer *x, size_t tokens, marin_buffer *out) {
    return guard([&] {
        if (x->dtype != MARIN_BF16) shape("matmul input element size", 2, dtype_bytes(x->dtype));
        if (out->dtype != MARIN_BF16) shape("matmul output element size", 2, dtype_bytes(out->dtype));
        check_len("matmul input", mul(tokens, w->cols, "matmul input"), x->len);
        check_len("matmul output", mul(tokens, w->rows, "matmul output"), out->len);
        if (!tokens || !w->rows || !w->cols) return;
        if (!gemv_supported(w)) unsupported("bf16 product layout (group and cols multiples of 64)", 64, w->group);
        const size_t need = product_scratch_bound(w, tokens);
        if (need > NOALLOC_SCRATCH_BYTES)
            unsupported("scratch bytes of an allocation-free product (tokens x columns too large)",
                        NOALLOC_SCRATCH_BYTES, need);
        void *ptr = scratch_on(g->device);
        GemvIn in;
        in.mode = IN_BF16;
        in.x = x->data;
        in.x_stride = w->cols;
        GemvOut o;
        o.mode = OUT_BF16;
        o.y = out->data;
        o.y_stride = w->rows;
        g->fixed_work = ptr;
        g->fixed_work_bytes = NOALLOC_SCRATCH_BYTES;
        try {
            launch_product(g, w, in, o, tokens);
        } catch (...) {
            g->fixed_work = nullptr;
            g->fixed_work_bytes = 0;
            throw;
        }
        g->fixed_work = nullptr;
        g->fixed_work_bytes = 0;
    });
}
