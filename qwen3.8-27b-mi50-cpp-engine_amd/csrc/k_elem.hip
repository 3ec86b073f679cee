// k_elem.hip -- RMSNorm + quantize rows, activation / weight quantizers, SwiGLU + quantize,
// the seeded synthetic generator, and the device plumbing of the C ABI.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "q27x_dev.h"
#include "q27x_int.h"

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
// One 256-thread block per row. Thread t owns elements 1024i + 4t + e (sum of squares in that
// order, four wave trees, ((w0+w1)+w2)+w3); nrm = x*inv*(plus+w); a group of 16 is 4 threads.
constexpr int kNormMaxChunks = 8;   // n <= 8192
__global__ __launch_bounds__(256) void k_norm(NormArgs a) {
    if (a.stop && *a.stop) return;
    const int r = blockIdx.x;
    const int rs = a.row_sel ? *a.row_sel : r;      // source row
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int n = a.n, nch = n >> 10;
    float xv[kNormMaxChunks][4];
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i) {
        if (i >= nch) break;
        const int k = i * 1024 + 4 * t;
        float v[4];
        if (a.emb) {
            const uint2 u = *(const uint2*)(a.emb + (size_t)a.tok[rs] * n + k);
            v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xFFFF0000u);
            v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xFFFF0000u);
        } else if (a.x_bf16) {
            const uint2 u = *(const uint2*)((const uint16_t*)a.x + (size_t)rs * a.xstride + k);
            v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xFFFF0000u);
            v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xFFFF0000u);
        } else {
            const float4 f = *(const float4*)((const float*)a.x + (size_t)rs * a.xstride + k);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        }
        if (a.hout) {   // head: the final residual row, bf16(bf16(r1) + r2) or bf16(r2)
            uint16_t hb[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float s = a.hadd ? bf2f(a.hadd[(size_t)rs * n + k + e]) + v[e] : v[e];
                hb[e] = f2bf(s);
                v[e] = bf2f(hb[e]);
            }
            *(uint2*)(a.hout + (size_t)r * n + k) = make_uint2((uint32_t)hb[0] | ((uint32_t)hb[1] << 16),
                                                              (uint32_t)hb[2] | ((uint32_t)hb[3] << 16));
        }
        if (a.hcopy) {
            *(uint2*)(a.hcopy + (size_t)r * n + k) =
                make_uint2((uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16),
                           (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16));
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[i][e] = v[e];
    }
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i) {
        if (i >= nch) break;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = __builtin_fmaf(xv[i][e], xv[i][e], acc);
    }
    __shared__ float wsum[4];
    acc = tree64(acc);
    if (lane == 0) wsum[wv] = acc;
    __syncthreads();
    const float ss = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
    const float inv = rsqrt_cr(ss * (1.0f / (float)n) + a.eps);
    const float g = 1.0f / a.in_scale;
#pragma unroll
    for (int i = 0; i < kNormMaxChunks; ++i) {
        if (i >= nch) break;
        const int k = i * 1024 + 4 * t;
        const uint2 wu = *(const uint2*)(a.w + k);
        const float wf[4] = { __uint_as_float(wu.x << 16), __uint_as_float(wu.x & 0xFFFF0000u),
                              __uint_as_float(wu.y << 16), __uint_as_float(wu.y & 0xFFFF0000u) };
        float nm[4];
        uint16_t yb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            nm[e] = xv[i][e] * inv * (a.plus + wf[e]);
            yb[e] = f2bf(nm[e]);
        }
        if (a.y)
            *(uint2*)(a.y + (size_t)r * a.ystride + k) = make_uint2((uint32_t)yb[0] | ((uint32_t)yb[1] << 16),
                                                                   (uint32_t)yb[2] | ((uint32_t)yb[3] << 16));
        if (a.xq) {
            float q[4], mx = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) { q[e] = a.quant_bf16 ? bf2f(yb[e]) : nm[e]; mx = fmaxf(mx, fabsf(q[e])); }
            mx = max_xor(mx, 4);
            const float s = mx * g * (1.0f / 127.0f);
            const float qi = (s > 0.0f) ? (g / s) : 0.0f;
            uint32_t pk = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) pk |= ((uint32_t)(uint8_t)qcode(q[e], qi)) << (8 * e);
            *(uint32_t*)(a.xq + (size_t)r * n + k) = pk;
            if ((t & 3) == 0) a.xs[(size_t)r * (n >> 4) + (k >> 4)] = s;
        }
    }
}
int launch_norm(const NormArgs& a, int nr, hipStream_t s) {
    if (a.n < 1024 || (a.n & 1023) || (a.n >> 10) > kNormMaxChunks || !a.w || nr < 1) {
        set_error("norm: n=%d must be a multiple of 1024 up to 8192", a.n);
        return Q27X_E_SHAPE;
    }
    hipLaunchKernelGGL(k_norm, dim3(nr), dim3(256), 0, s, a);
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
