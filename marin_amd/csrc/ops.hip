// Elementwise ops of the reference's backend API (crates/cuda/src/ops.rs:110-236, kernels.cu:51-175) on CDNA4.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <utility>

#include "ops.hpp"

namespace marin {

// RMSNorm of one row per block: src may equal dst. x * (1 / sqrtf(mean(x^2) + eps)) * w (kernels.cu:51-60).
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *__restrict__ src, float *dst,
                                                       const float *__restrict__ w, int dim, float eps) {
    const float *row = src + (size_t)blockIdx.x * dim;
    float *out = dst + (size_t)blockIdx.x * dim;
    __shared__ float red[4];
    float s = 0.0f;
    for (int i = threadIdx.x; i < dim; i += 256) s += row[i] * row[i];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = 1.0f / sqrtf(total / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += 256) out[i] = row[i] * scale * w[i];
}

void launch_rms_norm(marin_gpu *g, const float *src, float *dst, const float *w, size_t rows, size_t dim, float eps) {
    if (!rows) return;
    rms_norm_kernel<<<dim3((unsigned)rows), dim3(256), 0, g->stream>>>(src, dst, w, (int)dim, eps);
    g->launched();
}

// RoPE over [token][head][head_dim] (ops.rs:56-95 order: pairs (i, i + hd/2)); freq[i] = theta^(-2i/hd) comes from
// the host (the same powf the CPU path uses), the angles are position * freq with sincosf on the device.
__global__ void rope_kernel(float *__restrict__ x, const float *__restrict__ freq, int heads, int hd, uint32_t start) {
    const int token = blockIdx.x / heads;
    float *head = x + (size_t)blockIdx.x * hd;
    const int half = hd / 2;
    const float position = (float)(start + token);
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        float s, c;
        sincosf(position * freq[i], &s, &c);
        const float a = head[i], b = head[i + half];
        head[i] = a * c - b * s;
        head[i + half] = b * c + a * s;
    }
}

static std::mutex g_freq_mutex;
static std::map<std::pair<marin_gpu *, std::pair<int, uint32_t>>, float *> g_freq;

const float *rope_frequencies(marin_gpu *g, size_t hd, float theta) {
    uint32_t tb;
    std::memcpy(&tb, &theta, 4);
    std::lock_guard<std::mutex> lock(g_freq_mutex);
    auto key = std::make_pair(g, std::make_pair((int)hd, tb));
    auto it = g_freq.find(key);
    if (it != g_freq.end()) return it->second;
    std::vector<float> f(hd / 2);
    for (size_t i = 0; i < hd / 2; ++i) f[i] = powf(theta, -((float)i * 2.0f / (float)hd));
    float *d = (float *)g->alloc(std::max<size_t>(f.size(), 1) * 4, false);
    g->upload(d, f.data(), f.size() * 4);
    g_freq[key] = d;
    return d;
}

float *make_rope_frequencies(marin_gpu *g, size_t hd, float theta) {
    std::vector<float> f(hd / 2);
    for (size_t i = 0; i < hd / 2; ++i) f[i] = powf(theta, -((float)i * 2.0f / (float)hd));
    float *d = (float *)g->alloc(std::max<size_t>(f.size(), 1) * 4, false);
    g->upload(d, f.data(), f.size() * 4);
    return d;
}

// Cosine and sine of the RoPE angle pos * freq[i] for positions 0 .. positions - 1, [pos][hd/2] (the same sincosf
// of the same f32 angle that rope_kernel computes, so a table lookup gives the same bits).
__global__ void rope_table_kernel(const float *__restrict__ freq, int half, size_t positions, float2 *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= positions * half) return;
    const float position = (float)(i / half);
    float s, c;
    sincosf(position * freq[i % half], &s, &c);
    out[i] = make_float2(c, s);
}

float2 *make_rope_table(marin_gpu *g, const float *freq, size_t hd, size_t positions) {
    const size_t n = std::max<size_t>(positions, 1) * std::max<size_t>(hd / 2, 1);
    float2 *t = (float2 *)g->alloc(n * sizeof(float2), false);
    rope_table_kernel<<<(unsigned)((n + 255) / 256), 256, 0, g->stream>>>(freq, (int)(hd / 2),
                                                                           std::max<size_t>(positions, 1), t);
    g->launched();
    return t;
}

void forget_rope_frequencies(marin_gpu *g) {
    std::lock_guard<std::mutex> lock(g_freq_mutex);
    for (auto it = g_freq.begin(); it != g_freq.end();) {
        if (it->first.first == g) {
            g->release(it->second);
            it = g_freq.erase(it);
        } else {
            ++it;
        }
    }
}

void launch_rope(marin_gpu *g, float *x, size_t head_count, size_t heads, size_t hd, size_t start, float theta) {
    if (!head_count) return;
    const float *freq = rope_frequencies(g, hd, theta);
    rope_kernel<<<dim3((unsigned)head_count), dim3((unsigned)std::min<size_t>(std::max<size_t>(hd / 2, 1), 1024)), 0,
                  g->stream>>>(x, freq, (int)heads, (int)hd, (uint32_t)start);
    g->launched();
}

__global__ void silu_mul_kernel(float *__restrict__ gate, const float *__restrict__ up, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float g = gate[i];
        gate[i] = g / (1.0f + expf(-g)) * up[i];
    }
}

__global__ void add_kernel(float *__restrict__ a, const float *__restrict__ b, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) a[i] += b[i];
}

}  // namespace marin

using namespace marin;

static size_t rows_of(size_t len, size_t width, const char *what) {
    if (width == 0 || len % width != 0) shape(what, width, len);
    return len / width;
}

static void require_f32(const marin_buffer *b, const char *what) {
    if (b->dtype != MARIN_F32) shape(what, 4, dtype_bytes(b->dtype));
}

extern "C" {

marin_status marin_rms_norm(marin_gpu *g, marin_buffer *x, const marin_buffer *weight, float eps) {
    return guard([&] {
        require_f32(x, "rms_norm element size");
        const size_t rows = rows_of(x->len, weight->len, "rms_norm input");
        launch_rms_norm(g, (const float *)x->data, (float *)x->data, (const float *)weight->data, rows, weight->len,
                        eps);
    });
}

marin_status marin_rms_norm_into(marin_gpu *g, const marin_buffer *x, const marin_buffer *weight, marin_buffer *out,
                                 float eps) {
    return guard([&] {
        require_f32(x, "rms_norm element size");
        const size_t rows = rows_of(x->len, weight->len, "rms_norm input");
        check_len("rms_norm output", x->len, out->len);
        launch_rms_norm(g, (const float *)x->data, (float *)out->data, (const float *)weight->data, rows, weight->len,
                        eps);
    });
}

marin_status marin_rope(marin_gpu *g, marin_buffer *x, size_t heads, size_t head_dim, size_t start, float theta) {
    return guard([&] {
        if (head_dim == 0 || head_dim % 2 != 0 || heads == 0) shape("rope head layout", 2, head_dim);
        const size_t per_token = mul(heads, head_dim, "rope");
        const size_t head_count = rows_of(x->len, head_dim, "rope input");
        rows_of(x->len, per_token, "rope input");
        require_f32(x, "rope element size");
        launch_rope(g, (float *)x->data, head_count, heads, head_dim, start, theta);
    });
}

marin_status marin_silu_mul(marin_gpu *g, marin_buffer *gate, const marin_buffer *up) {
    return guard([&] {
        check_len("silu_mul operands", gate->len, up->len);
        if (!gate->len) return;
        silu_mul_kernel<<<dim3((unsigned)((gate->len + 255) / 256)), dim3(256), 0, g->stream>>>(
            (float *)gate->data, (const float *)up->data, gate->len);
        g->launched();
    });
}

marin_status marin_add(marin_gpu *g, marin_buffer *a, const marin_buffer *b) {
    return guard([&] {
        check_len("add operands", a->len, b->len);
        if (!a->len) return;
        add_kernel<<<dim3((unsigned)((a->len + 255) / 256)), dim3(256), 0, g->stream>>>((float *)a->data,
                                                                                       (const float *)b->data, a->len);
        g->launched();
    });
}

}  // extern "C"
