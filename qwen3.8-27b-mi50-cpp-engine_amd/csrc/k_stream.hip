// k_stream.hip -- HBM calibration kernels: a streaming read and a plain copy of a known number of
// bytes. They give the achievable read bandwidth that the projection kernels are compared with,
// and the reference launch for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE counters.
#include <vector>

#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

// Each thread keeps U 16-byte loads in flight per iteration; consecutive threads read consecutive
// 16-byte words, so a wave reads U contiguous KiB-runs. The xor of everything read goes to one
// word per block so the loads cannot be dropped.
template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ p, size_t n16, uint32_t* out) {
    const size_t nt = (size_t)gridDim.x * 256;
    uint32_t acc = 0u;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += nt * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t j = i + (size_t)u * nt;
            v[u] = (j < n16) ? ld_nt16(p + j) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    __shared__ uint32_t sred[4];
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
    if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = sred[0] ^ sred[1] ^ sred[2] ^ sred[3];
}

__global__ __launch_bounds__(256) void k_stream_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
    const size_t nt = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += nt * 4) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const size_t j = i + (size_t)u * nt;
            v[u] = (j < n16) ? ld_nt16(src + j) : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const size_t j = i + (size_t)u * nt;
            if (j < n16) dst[j] = v[u];
        }
    }
}

static int cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
    return n;
}

}  // namespace q27x

using namespace q27x;

extern "C" int q27x_bench_stream(int mode, size_t bytes, int blocks_per_cu, int unroll, int iters, float* ms) {
    if (!ms || (mode != 0 && mode != 1) || bytes < 4096 || (bytes & 15) || blocks_per_cu < 1 || blocks_per_cu > 64 ||
        iters < 1 || !(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8)) {
        set_error("q27x_bench_stream: bad arguments");
        return Q27X_E_ARG;
    }
    // enough distinct sections that a section is out of the 256 MB Infinity Cache when revisited
    const size_t span = (size_t)1 << 30;
    const int nsec = (int)((span + bytes - 1) / bytes) < 2 ? 2 : (int)((span + bytes - 1) / bytes);
    const size_t total = (size_t)nsec * bytes;
    char* buf = nullptr;
    char* dst = nullptr;
    uint32_t* out = nullptr;
    const int grid = cu_count() * blocks_per_cu;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = Q27X_OK;
    auto fail = [&](hipError_t e, const char* what) { rc = hip_fail(e, what); };
    hipError_t e;
    if ((e = hipMalloc(&buf, total)) != hipSuccess) { fail(e, "hipMalloc"); goto done; }
    if (mode == 1 && (e = hipMalloc(&dst, bytes)) != hipSuccess) { fail(e, "hipMalloc"); goto done; }
    if ((e = hipMalloc(&out, (size_t)grid * 4)) != hipSuccess) { fail(e, "hipMalloc"); goto done; }
    if ((e = hipMemset(buf, 0x5A, total)) != hipSuccess) { fail(e, "hipMemset"); goto done; }
    if ((e = hipEventCreate(&e0)) != hipSuccess || (e = hipEventCreate(&e1)) != hipSuccess) { fail(e, "hipEventCreate"); goto done; }
    {
        const size_t n16 = bytes / 16;
        auto launch = [&](int i) {
            const uint4* p = (const uint4*)(buf + (size_t)(i % nsec) * bytes);
            if (mode == 1) hipLaunchKernelGGL(k_stream_copy, dim3(grid), dim3(256), 0, nullptr, p, (uint4*)dst, n16);
            else if (unroll == 1) hipLaunchKernelGGL(k_stream_read<1>, dim3(grid), dim3(256), 0, nullptr, p, n16, out);
            else if (unroll == 2) hipLaunchKernelGGL(k_stream_read<2>, dim3(grid), dim3(256), 0, nullptr, p, n16, out);
            else if (unroll == 4) hipLaunchKernelGGL(k_stream_read<4>, dim3(grid), dim3(256), 0, nullptr, p, n16, out);
            else hipLaunchKernelGGL(k_stream_read<8>, dim3(grid), dim3(256), 0, nullptr, p, n16, out);
        };
        for (int i = 0; i < 2; ++i) launch(i);
        if ((e = hipEventRecord(e0, nullptr)) != hipSuccess) { fail(e, "hipEventRecord"); goto done; }
        for (int i = 0; i < iters; ++i) launch(i + 2);
        if ((e = hipEventRecord(e1, nullptr)) != hipSuccess) { fail(e, "hipEventRecord"); goto done; }
        if ((e = hipEventSynchronize(e1)) != hipSuccess) { fail(e, "hipEventSynchronize"); goto done; }
        float t = 0.0f;
        if ((e = hipEventElapsedTime(&t, e0, e1)) != hipSuccess) { fail(e, "hipEventElapsedTime"); goto done; }
        *ms = t / (float)iters;
        if ((e = hipGetLastError()) != hipSuccess) { fail(e, "k_stream"); goto done; }
    }
done:
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (buf) (void)hipFree(buf);
    if (dst) (void)hipFree(dst);
    if (out) (void)hipFree(out);
    return rc;
}
