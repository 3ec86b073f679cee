// k_elem.hip -- RMSNorm + quantize rows, activation / weight quantizers, SwiGLU + quantize,
// the seeded synthetic generator, and the device plumbing of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "q27x_dev.h"
#include "q27x_int.h"
#include "q27x_norm.h"

namespace q27x {

// ---------------------------------------------------------------- errors
static thread_local char g_err[512] = "";
void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
int hip_fail(hipError_t e, const char* what) {
    set_error("HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
    return e == hipErrorOutOfMemory ? Q27X_E_NOMEM : Q27X_E_HIP;
}

// ---------------------------------------------------------------- RMSNorm + quantize
// One 256-thread block per row, in the canonical order of norm_rows (q27x_norm.h).
constexpr int kNormMaxChunks = 8;   // n <= 8192
template <int NCH>
__global__ __launch_bounds__(256) void k_norm(NormArgs a) {
    if (stopped(a.stop)) return;
    if (a.stamp && blockIdx.x == 0 && threadIdx.x == 0) *a.stamp = __builtin_amdgcn_s_memrealtime();
    __shared__ float wsum[1][4];
    norm_rows<NCH, 1>(a, blockIdx.x, 1, wsum);
}
int launch_norm(const NormArgs& a, int nr, hipStream_t s) {
    if (a.n < 1024 || (a.n & 1023) || (a.n >> 10) > kNormMaxChunks || !a.w || nr < 1) {
        set_error("norm: n=%d must be a multiple of 1024 up to 8192", a.n);
        return Q27X_E_SHAPE;
    }
    switch (a.n >> 10) {
        case 1: hipLaunchKernelGGL(k_norm<1>, dim3(nr), dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL(k_norm<2>, dim3(nr), dim3(256), 0, s, a); break;
        case 3: hipLaunchKernelGGL(k_norm<3>, dim3(nr), dim3(256), 0, s, a); break;
        case 4: hipLaunchKernelGGL(k_norm<4>, dim3(nr), dim3(256), 0, s, a); break;
        case 5: hipLaunchKernelGGL(k_norm<5>, dim3(nr), dim3(256), 0, s, a); break;
        case 6: hipLaunchKernelGGL(k_norm<6>, dim3(nr), dim3(256), 0, s, a); break;
        case 7: hipLaunchKernelGGL(k_norm<7>, dim3(nr), dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL(k_norm<8>, dim3(nr), dim3(256), 0, s, a); break;
    }
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// ---------------------------------------------------------------- R5 activation quantizer
__global__ __launch_bounds__(256) void k_quant_rows(const uint16_t* __restrict__ x, int xstride, int8_t* __restrict__ xq,
                                                    int qstride, float* __restrict__ xs, int sstride, int n, float g) {
    const int r = blockIdx.y;
    const int gi = blockIdx.x * 256 + threadIdx.x;
    const int k0 = gi * 16;
    if (k0 >= n) return;
    const uint16_t* xr = x + (size_t)r * xstride + k0;
    float v[16], mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) { v[j] = bf2f(xr[j]); mx = fmaxf(mx, fabsf(v[j])); }
    const float s = mx * g * (1.0f / 127.0f);
    const float inv = (s > 0.0f) ? (g / s) : 0.0f;
    xs[(size_t)r * sstride + gi] = s;
    int8_t* q = xq + (size_t)r * qstride + k0;
#pragma unroll
    for (int j = 0; j < 16; ++j) q[j] = qcode(v[j], inv);
}
int launch_quant_rows(const uint16_t* x, int xstride, int8_t* xq, int qstride, float* xs, int sstride, int n,
                      float in_scale, int nrows, hipStream_t s) {
    if (!x || !xq || !xs || n < 16 || (n & 15) || nrows < 1 || !(in_scale > 0.0f)) {
        set_error("quant_rows: bad arguments (n=%d nrows=%d)", n, nrows);
        return Q27X_E_ARG;
    }
    const int groups = n >> 4;
    hipLaunchKernelGGL(k_quant_rows, dim3((groups + 255) / 256, nrows), dim3(256), 0, s, x, xstride, xq, qstride, xs,
                       sstride, n, 1.0f / in_scale);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// ---------------------------------------------------------------- R16 SwiGLU + quantize
__global__ __launch_bounds__(256) void k_swiglu(const float* __restrict__ G, const float* __restrict__ U, int stride,
                                                int8_t* __restrict__ xq, float* __restrict__ xs, int n, float gs) {
    const int r = blockIdx.y;
    const int gi = blockIdx.x * 256 + threadIdx.x;
    if (gi * 16 >= n) return;
    const size_t base = (size_t)r * stride + (size_t)gi * 16;
    float v[16], mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float a = G[base + j];
        const float sw = a / (1.0f + qexp(-a));
        v[j] = sw * U[base + j] * gs;
        mx = fmaxf(mx, fabsf(v[j]));
    }
    const float sc = mx * (1.0f / 127.0f);
    const float inv = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
    xs[(size_t)r * (n >> 4) + gi] = sc;
#pragma unroll
    for (int j = 0; j < 16; ++j) xq[(size_t)r * n + (size_t)gi * 16 + j] = qcode(v[j], inv);
}
int launch_swiglu(const float* g, const float* u, int stride, int8_t* xq, float* xs, int n, float in_scale, int nr,
                  hipStream_t s) {
    if (!g || !u || !xq || !xs || n < 16 || (n & 15) || nr < 1 || !(in_scale > 0.0f)) {
        set_error("swiglu: bad arguments");
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_swiglu, dim3((n / 16 + 255) / 256, nr), dim3(256), 0, s, g, u, stride, xq, xs, n,
                       1.0f / in_scale);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// ---------------------------------------------------------------- R8 weight quantizer / generator
// One thread per group of 64: sc = mx/127, q = rint(v/sc) (src/q27_nvfp4.hip:4259-4289).
__global__ __launch_bounds__(256) void k_quant_w(const float* __restrict__ w, int rows, int K, int8_t* __restrict__ wq,
                                                 float* __restrict__ ws) {
    const long long gi = (long long)blockIdx.x * 256 + threadIdx.x;
    const int ng = K >> 6;
    if (gi >= (long long)rows * ng) return;
    const float* src = w + (size_t)gi * 64;
    float mx = 0.0f;
    for (int j = 0; j < 64; ++j) mx = fmaxf(mx, fabsf(src[j]));
    const float sc = mx * (1.0f / 127.0f);
    const float inv = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
    ws[gi] = sc;
    for (int j = 0; j < 64; ++j) wq[(size_t)gi * 64 + j] = qcode(src[j], inv);
}
int launch_quant_w(const float* w, int rows, int K, int8_t* wq, float* ws, hipStream_t s) {
    if (!w || !wq || !ws || rows < 1 || K < 64 || (K & 63)) { set_error("quant_w: bad arguments"); return Q27X_E_ARG; }
    const long long ng = (long long)rows * (K >> 6);
    hipLaunchKernelGGL(k_quant_w, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, s, w, rows, K, wq, ws);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// Synthetic int8 projection: logical element (r, k) of tensor `key` is N(0, 0.02) from the
// counter-based generator, quantized per 64. layout_gu places logical row r of a gate (is_up=0)
// or up (is_up=1) matrix at physical row (r/16)*32 + (r%16) + 16*is_up (16-row interleave).
__global__ __launch_bounds__(256) void k_gen_i8(int8_t* __restrict__ W, float* __restrict__ WS, int rows, int K,
                                                uint64_t key, int layout_gu, int is_up) {
    const long long gi = (long long)blockIdx.x * 256 + threadIdx.x;
    const int ng = K >> 6;
    if (gi >= (long long)rows * ng) return;
    const int r = (int)(gi / ng), gg = (int)(gi - (long long)r * ng);
    const int pr = layout_gu ? (r / 16) * 32 + (r % 16) + 16 * is_up : r;
    float v[64], mx = 0.0f;
    const uint64_t base = (uint64_t)r * (uint64_t)K + (uint64_t)gg * 64;
#pragma unroll 8
    for (int j = 0; j < 64; ++j) { v[j] = normal_k(key, base + j) * 0.02f; mx = fmaxf(mx, fabsf(v[j])); }
    const float sc = mx * (1.0f / 127.0f);
    const float inv = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
    WS[(size_t)pr * ng + gg] = sc;
    int8_t* dst = W + (size_t)pr * K + (size_t)gg * 64;
#pragma unroll
    for (int j = 0; j < 64; j += 4) {
        const uint32_t pk = (uint32_t)(uint8_t)qcode(v[j], inv) | ((uint32_t)(uint8_t)qcode(v[j + 1], inv) << 8) |
                            ((uint32_t)(uint8_t)qcode(v[j + 2], inv) << 16) | ((uint32_t)(uint8_t)qcode(v[j + 3], inv) << 24);
        *(uint32_t*)(dst + j) = pk;
    }
}
int launch_gen_i8(int8_t* W, float* WS, int rows, int K, uint64_t key, int layout_gu, int is_up, hipStream_t s) {
    const long long ng = (long long)rows * (K >> 6);
    hipLaunchKernelGGL(k_gen_i8, dim3((unsigned)((ng + 255) / 256)), dim3(256), 0, s, W, WS, rows, K, key, layout_gu,
                       is_up);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
__global__ __launch_bounds__(256) void k_gen_bf16(uint16_t* __restrict__ p, size_t n, uint64_t key, float stdv,
                                                  float mean, int uniform) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float v = uniform ? uniform_k(key, i) * stdv : mean + normal_k(key, i) * stdv;
        p[i] = f2bf(v);
    }
}
int launch_gen_bf16(uint16_t* p, size_t n, uint64_t key, float stdv, float mean, int uniform, hipStream_t s) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_gen_bf16, dim3((unsigned)blocks), dim3(256), 0, s, p, n, key, stdv, mean, uniform);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

__global__ void k_math_test(const float* __restrict__ x, float* __restrict__ y, int n, int op) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    float r;
    switch (op) {
        case 0: r = qexp(v); break;
        case 1: r = qexp2(v); break;
        case 2: r = qlog1p(v); break;
        case 3: r = qsigmoid(v); break;
        case 4: r = qsilu(v); break;
        default: r = qsoftplus(v); break;
    }
    y[i] = r;
}
int launch_math_test(const float* x, float* y, int n, int op, hipStream_t s) {
    hipLaunchKernelGGL(k_math_test, dim3((n + 255) / 256), dim3(256), 0, s, x, y, n, op);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

}  // namespace q27x

// ---------------------------------------------------------------- C ABI: errors and plumbing
using namespace q27x;
extern "C" {
const char* q27x_last_error(void) { return g_err; }
const char* q27x_version(void) { return "q27x 0.1 gfx950"; }
int q27x_device_count(int* n) {
    if (!n) return Q27X_E_ARG;
    int c = 0;
    const hipError_t e = hipGetDeviceCount(&c);
    if (e != hipSuccess) { *n = 0; return hip_fail(e, "hipGetDeviceCount"); }
    *n = c;
    return Q27X_OK;
}
int q27x_set_device(int dev) { Q27X_HIP(hipSetDevice(dev)); return Q27X_OK; }
int q27x_device_name(int dev, char* buf, int len) {
    hipDeviceProp_t p;
    Q27X_HIP(hipGetDeviceProperties(&p, dev));
    if (buf && len > 0) { snprintf(buf, (size_t)len, "%s (%s)", p.name, p.gcnArchName); }
    return Q27X_OK;
}
int q27x_device_cus(int dev, int* n_cu) {
    hipDeviceProp_t p;
    Q27X_HIP(hipGetDeviceProperties(&p, dev));
    if (n_cu) *n_cu = p.multiProcessorCount;
    return Q27X_OK;
}
int q27x_malloc(void** p, size_t bytes) { if (!p) return Q27X_E_ARG; Q27X_HIP(hipMalloc(p, bytes ? bytes : 1)); return Q27X_OK; }
int q27x_free(void* p) { Q27X_HIP(hipFree(p)); return Q27X_OK; }
int q27x_host_malloc(void** p, size_t bytes) { if (!p) return Q27X_E_ARG; Q27X_HIP(hipHostMalloc(p, bytes ? bytes : 1, hipHostMallocDefault)); return Q27X_OK; }
int q27x_host_free(void* p) { Q27X_HIP(hipHostFree(p)); return Q27X_OK; }
int q27x_memcpy_h2d(void* dst, const void* src, size_t bytes, q27x_stream_t s) {
    Q27X_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)s));
    Q27X_HIP(hipStreamSynchronize((hipStream_t)s));
    return Q27X_OK;
}
int q27x_memcpy_d2h(void* dst, const void* src, size_t bytes, q27x_stream_t s) {
    Q27X_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)s));
    Q27X_HIP(hipStreamSynchronize((hipStream_t)s));
    return Q27X_OK;
}
int q27x_memcpy_d2d(void* dst, const void* src, size_t bytes, q27x_stream_t s) {
    Q27X_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)s));
    return Q27X_OK;
}
int q27x_memset(void* p, int value, size_t bytes, q27x_stream_t s) {
    Q27X_HIP(hipMemsetAsync(p, value, bytes, (hipStream_t)s));
    return Q27X_OK;
}
int q27x_stream_create(q27x_stream_t* s) {
    if (!s) return Q27X_E_ARG;
    hipStream_t st;
    Q27X_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
    *s = (q27x_stream_t)st;
    return Q27X_OK;
}
int q27x_stream_destroy(q27x_stream_t s) { Q27X_HIP(hipStreamDestroy((hipStream_t)s)); return Q27X_OK; }
int q27x_stream_sync(q27x_stream_t s) { Q27X_HIP(hipStreamSynchronize((hipStream_t)s)); return Q27X_OK; }
int q27x_device_sync(void) { Q27X_HIP(hipDeviceSynchronize()); return Q27X_OK; }
int q27x_event_create(void** e) {
    if (!e) return Q27X_E_ARG;
    hipEvent_t ev;
    Q27X_HIP(hipEventCreate(&ev));
    *e = (void*)ev;
    return Q27X_OK;
}
int q27x_event_destroy(void* e) { Q27X_HIP(hipEventDestroy((hipEvent_t)e)); return Q27X_OK; }
int q27x_event_record(void* e, q27x_stream_t s) { Q27X_HIP(hipEventRecord((hipEvent_t)e, (hipStream_t)s)); return Q27X_OK; }
int q27x_event_elapsed_ms(void* a, void* b, float* ms) {
    if (!ms) return Q27X_E_ARG;
    Q27X_HIP(hipEventSynchronize((hipEvent_t)b));
    Q27X_HIP(hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b));
    return Q27X_OK;
}

// ---------------------------------------------------------------- C ABI: kernel tier
int q27x_quant_rows(const uint16_t* x, int xstride, int8_t* xq, int qstride, float* xs, int sstride, int n,
                    float in_scale, int nrows, q27x_stream_t s) {
    return launch_quant_rows(x, xstride, xq, qstride, xs, sstride, n, in_scale, nrows, (hipStream_t)s);
}
int q27x_quant_weights_i8g64(const float* w, int rows, int K, int8_t* wq, float* ws, q27x_stream_t s) {
    return launch_quant_w(w, rows, K, wq, ws, (hipStream_t)s);
}
int q27x_rmsnorm_quant_rows(const void* x, int x_bf16, int xstride, const uint16_t* w, float plus, float eps, int n,
                            uint16_t* hcopy, uint16_t* y, int ystride, int8_t* xq, float* xs, int quant_bf16,
                            float in_scale, int nr, q27x_stream_t s) {
    if (!x || (xq && !xs) || !(in_scale > 0.0f)) { set_error("q27x_rmsnorm_quant_rows: bad arguments"); return Q27X_E_ARG; }
    NormArgs a{};
    a.x = x; a.x_bf16 = x_bf16 ? 1 : 0; a.xstride = xstride; a.w = w; a.plus = plus; a.eps = eps; a.n = n;
    a.hcopy = hcopy; a.y = y; a.ystride = ystride; a.xq = xq; a.xs = xs; a.quant_bf16 = quant_bf16 ? 1 : 0;
    a.in_scale = in_scale;
    return launch_norm(a, nr, (hipStream_t)s);
}
int q27x_swiglu_quant_rows(const float* gate, const float* up, int stride, int8_t* xq, float* xs, int n,
                           float in_scale, int nr, q27x_stream_t s) {
    return launch_swiglu(gate, up, stride, xq, xs, n, in_scale, nr, (hipStream_t)s);
}
int q27x_math_test(const float* x, float* y, int n, int op, q27x_stream_t s) {
    if (!x || !y || n < 0) return Q27X_E_ARG;
    return launch_math_test(x, y, n, op, (hipStream_t)s);
}
}  // extern "C"
