// k_prefill.hip -- the element kernels of the layer-major prefill (ls_q8_layer's stages,
// src/q27_main.cpp:4076-4316) around the int8 MFMA GEMM: the per-(token, group) quantizer of bf16
// rows, the GDN chunk conv, the GDN row scalars and the SwiGLU quantizer. Each keeps the decode
// path's arithmetic for its values, so a prefilled state continues exactly like a decoded one.
#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

// bf16 rows [M][ld] -> per-(token, group) codes [M][K] and scales [M][K / gs] (the quantizer of
// k_quant_tok_grp on the rows' float values with gq = 1/in_scale: sc = max|v| gq / 127,
// qi = sc > 0 ? gq / sc : 0).
// One 256-thread block per (group, token), four values per thread per 1024 columns.
__global__ __launch_bounds__(256) void k_pf_quant_bf16(const uint16_t* __restrict__ x, int ld, int K, int gs,
                                                       int8_t* __restrict__ xq, float* __restrict__ xs, float gq) {
    const int g = blockIdx.x, tok = blockIdx.y, t = threadIdx.x, ng = K / gs;
    __shared__ float red[4];
    const uint16_t* row = x + (size_t)tok * ld + (size_t)g * gs;
    float mx = 0.0f;
    for (int k = 4 * t; k < gs; k += 1024) {
        const uint2 u = *(const uint2*)(row + k);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(__uint_as_float(u.x << 16)), fabsf(__uint_as_float(u.x & 0xFFFF0000u))),
                             fmaxf(fabsf(__uint_as_float(u.y << 16)), fabsf(__uint_as_float(u.y & 0xFFFF0000u)))));
    }
    mx = max_xor(mx, 64);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = m * gq * (1.0f / 127.0f), qi = (sc > 0.0f) ? gq / sc : 0.0f;
    if (t == 0) xs[(size_t)tok * ng + g] = sc;
    int8_t* out = xq + (size_t)tok * K + (size_t)g * gs;
    for (int k = 4 * t; k < gs; k += 1024) {
        const uint2 u = *(const uint2*)(row + k);
        const uint32_t pk = (uint32_t)(uint8_t)qcode(__uint_as_float(u.x << 16), qi) |
                            ((uint32_t)(uint8_t)qcode(__uint_as_float(u.x & 0xFFFF0000u), qi) << 8) |
                            ((uint32_t)(uint8_t)qcode(__uint_as_float(u.y << 16), qi) << 16) |
                            ((uint32_t)(uint8_t)qcode(__uint_as_float(u.y & 0xFFFF0000u), qi) << 24);
        *(uint32_t*)(out + k) = pk;
    }
}
int launch_pf_quant_bf16(const uint16_t* x, int ld, int M, int K, int gs, float in_scale, int8_t* xq, float* xs,
                         hipStream_t s) {
    if (!x || !xq || !xs || M < 1 || K < 4 || gs < 4 || (gs & 3) || (K % gs) || ld < K || (ld & 3) || ((uintptr_t)x & 7) ||
        !(in_scale > 0.0f)) {
        set_error("prefill quant: bad arguments (M %d, K %d, gs %d, ld %d)", M, K, gs, ld);
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_pf_quant_bf16, dim3((unsigned)(K / gs), (unsigned)M), dim3(256), 0, s, x, ld, K, gs, xq, xs,
                       1.0f / in_scale);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// GDN conv of a chunk: the decode path's conv (k_gdn_conv_tp_tile, src/q27_gdn.hip:411-439: taps
// 0..3 over the three inputs before the row's and the row's own, the first a plain product, SiLU,
// bf16) of the q|k|v columns of the projection rows buf [C][ld] into out [C][ldo]. Each output
// depends only on raw inputs, so one thread per (channel, row): the inputs before row 0 come from
// the channel's 32-byte record (committed h0 h1 h2, then the npend pending raw inputs of the last
// decode call). k_pf_conv_commit then leaves the chunk's last three inputs in the record as the
// committed history, nothing pending.
__device__ __forceinline__ uint32_t conv_hist_at(const uint16_t* rec, int c, int npend, int j) {
    // element j (0..2) of the committed history after applying the npend pending inputs
    const int src = j + npend;                      // index into h0 h1 h2 r0 r1 ...
    return src < 3 ? rec[(size_t)c * 16 + src] : rec[(size_t)c * 16 + 4 + (src - 3)];
}
__global__ __launch_bounds__(256) void k_pf_conv(const uint16_t* __restrict__ buf, int ld, int C, int nconv,
                                                 const uint16_t* __restrict__ conv_w, const uint16_t* __restrict__ rec,
                                                 int npend, uint16_t* __restrict__ out, int ldo) {
    const int c = blockIdx.x * 256 + threadIdx.x, n = blockIdx.y;
    if (c >= nconv) return;
    uint32_t x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = n - 3 + j;                    // row of tap j; r < 0: the history
        x[j] = (r >= 0) ? buf[(size_t)r * ld + c] : conv_hist_at(rec, c, npend, 3 + r);
    }
    const uint2 wv = *(const uint2*)(conv_w + (size_t)c * 4);
    float acc = __uint_as_float(x[0] << 16) * __uint_as_float(wv.x << 16);
    acc = __builtin_fmaf(__uint_as_float(x[1] << 16), __uint_as_float(wv.x & 0xFFFF0000u), acc);
    acc = __builtin_fmaf(__uint_as_float(x[2] << 16), __uint_as_float(wv.y << 16), acc);
    acc = __builtin_fmaf(__uint_as_float(x[3] << 16), __uint_as_float(wv.y & 0xFFFF0000u), acc);
    out[(size_t)n * ldo + c] = f2bf(qsilu(acc));
}
__global__ __launch_bounds__(256) void k_pf_conv_commit(const uint16_t* __restrict__ buf, int ld, int C, int nconv,
                                                        uint16_t* __restrict__ rec, int npend) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= nconv) return;
    uint32_t h[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const int r = C - 3 + j;
        h[j] = (r >= 0) ? buf[(size_t)r * ld + c] : conv_hist_at(rec, c, npend, 3 + r);
    }
    uint4* d = (uint4*)(rec + (size_t)c * 16);
    d[0] = make_uint4(h[0] | (h[1] << 16), h[2], 0u, 0u);
    d[1] = make_uint4(0u, 0u, 0u, 0u);
}
int launch_pf_conv(const uint16_t* buf, int ld, int C, int nconv, const uint16_t* conv_w, uint16_t* rec, int npend,
                   uint16_t* out, int ldo, hipStream_t s) {
    if (!buf || !conv_w || !rec || !out || C < 1 || nconv < 1 || ld < nconv || ldo < nconv || npend < 0 ||
        npend > kMaxRows || ((uintptr_t)rec & 15) || ((uintptr_t)conv_w & 7)) {
        set_error("prefill conv: bad arguments");
        return Q27X_E_ARG;
    }
    const unsigned gx = (unsigned)((nconv + 255) / 256);
    hipLaunchKernelGGL(k_pf_conv, dim3(gx, (unsigned)C), dim3(256), 0, s, buf, ld, C, nconv, conv_w, rec, npend, out,
                       ldo);
    Q27X_HIP(hipGetLastError());
    // (after every row has read the record)
    hipLaunchKernelGGL(k_pf_conv_commit, dim3(gx), dim3(256), 0, s, buf, ld, C, nconv, rec, npend);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// GDN row scalars of C rows: the bf16 GEMV of in_a / in_b row h with each bf16 normed row y (the
// decode path's order: 8-element chunk c on lane c % 64 in ascending c, fmaf per element, the
// shfl tree, bf16 rounding; k_bf16_gemv2_tile, src/q27_util.hip:114-167), then
// decay = exp(-exp(A_log) softplus(a + dt_bias)) and beta = sigmoid(b) (src/q27_gdn.hip:206-372)
// into out [2][C][vh]. A block stages kAbTok rows y in LDS; each wave holds one weight row's
// chunks in registers (lane l: chunks l, l + 64, ...) and runs it against every staged row.
constexpr int kAbTok = 8;            // rows per block
constexpr int kAbChunks = 10;        // weight chunks per lane at most (K <= 5120)
// KC: chunks per lane (every lane runs KC of them; chunks past K / 8 have zero weights, and
// fma(0, x, acc) = acc for the finite normed rows, so they change nothing)
template <int KC>
__global__ __launch_bounds__(1024) void k_pf_ab(const uint16_t* __restrict__ in_a, const uint16_t* __restrict__ in_b,
                                                const uint16_t* __restrict__ A_log,
                                                const uint16_t* __restrict__ dt_bias, const uint16_t* __restrict__ y,
                                                int ystride, int K, int vh, int C, float* __restrict__ out) {
    extern __shared__ uint4 sy[];                 // [kAbTok][K / 8] chunks
    const int t0 = blockIdx.x * kAbTok, nt = (C - t0 < kAbTok) ? C - t0 : kAbTok;
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nch = K >> 3;
    for (int i = threadIdx.x; i < nt * nch; i += 1024) {
        const int n = i / nch, c = i - n * nch;
        sy[i] = *(const uint4*)(y + (size_t)(t0 + n) * ystride + 8 * c);
    }
    __syncthreads();
    for (int j = wv; j < 2 * vh; j += 16) {
        const int which = j / vh, head = j - which * vh;
        const uint16_t* wrow = (which ? in_b : in_a) + (size_t)head * K;
        uint4 w[KC];
#pragma unroll
        for (int i = 0; i < KC; ++i) {
            const int c = lane + 64 * i;
            w[i] = *(const uint4*)(wrow + 8 * (c < nch ? c : 0));
            if (c >= nch) w[i] = make_uint4(0u, 0u, 0u, 0u);
        }
        const float Aexp = which ? 0.0f : qexp(bf2f(A_log[head]));
        const float dtb = which ? 0.0f : bf2f(dt_bias[head]);
        for (int n = 0; n < nt; ++n) {
            const uint4* yr = sy + (size_t)n * nch;
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < KC; ++i) {
                const int c = lane + 64 * i;
                const uint4 x = yr[c < nch ? c : 0];
                acc = __builtin_fmaf(__uint_as_float(w[i].x << 16), __uint_as_float(x.x << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w[i].x & 0xFFFF0000u), __uint_as_float(x.x & 0xFFFF0000u), acc);
                acc = __builtin_fmaf(__uint_as_float(w[i].y << 16), __uint_as_float(x.y << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w[i].y & 0xFFFF0000u), __uint_as_float(x.y & 0xFFFF0000u), acc);
                acc = __builtin_fmaf(__uint_as_float(w[i].z << 16), __uint_as_float(x.z << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w[i].z & 0xFFFF0000u), __uint_as_float(x.z & 0xFFFF0000u), acc);
                acc = __builtin_fmaf(__uint_as_float(w[i].w << 16), __uint_as_float(x.w << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w[i].w & 0xFFFF0000u), __uint_as_float(x.w & 0xFFFF0000u), acc);
            }
            const float v = bfr(bcast0(tree64(acc)));
            if (lane == 0) {
                const float r = which ? qsigmoid(v) : qexp(-(Aexp * qsoftplus(v + dtb)));
                out[((size_t)which * C + t0 + n) * vh + head] = r;
            }
        }
    }
}
int launch_pf_ab(const uint16_t* in_a, const uint16_t* in_b, const uint16_t* A_log, const uint16_t* dt_bias,
                 const uint16_t* y, int ystride, int K, int vh, int C, float* out, hipStream_t s) {
    if (!in_a || !in_b || !A_log || !dt_bias || !y || !out || (K & 7) || K < 8 || K > 8 * 64 * kAbChunks || vh < 1 ||
        C < 1 || (ystride & 7) || ((uintptr_t)y & 15) || ((uintptr_t)in_a & 15) || ((uintptr_t)in_b & 15)) {
        set_error("prefill a/b: bad arguments");
        return Q27X_E_ARG;
    }
    const size_t lds = (size_t)kAbTok * (K / 8) * 16;
    static bool lds_set = false;
    const int mx = kAbTok * 64 * kAbChunks * 16;
    if (!lds_set) {
        Q27X_HIP(hipFuncSetAttribute((const void*)k_pf_ab<2>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_pf_ab<4>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_pf_ab<8>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        Q27X_HIP(hipFuncSetAttribute((const void*)k_pf_ab<10>, hipFuncAttributeMaxDynamicSharedMemorySize, mx));
        lds_set = true;
    }
    const int kc = (K / 8 + 63) / 64;
    const dim3 grid((unsigned)((C + kAbTok - 1) / kAbTok));
    if (kc <= 2) hipLaunchKernelGGL(k_pf_ab<2>, grid, dim3(1024), lds, s, in_a, in_b, A_log, dt_bias, y, ystride, K, vh, C, out);
    else if (kc <= 4) hipLaunchKernelGGL(k_pf_ab<4>, grid, dim3(1024), lds, s, in_a, in_b, A_log, dt_bias, y, ystride, K, vh, C, out);
    else if (kc <= 8) hipLaunchKernelGGL(k_pf_ab<8>, grid, dim3(1024), lds, s, in_a, in_b, A_log, dt_bias, y, ystride, K, vh, C, out);
    else hipLaunchKernelGGL(k_pf_ab<10>, grid, dim3(1024), lds, s, in_a, in_b, A_log, dt_bias, y, ystride, K, vh, C, out);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// SwiGLU of the fused gate|up GEMM rows gu [C][2I] (units of 32 rows: 16 gate rows, then the 16
// matching up rows) and the per-(token, group) quantizer of its I outputs: v = silu(g) u gscale
// with the decode path's expression (g / (1 + e^-g)), then sc = max|v| / 127 over each group of
// gs outputs. One 256-thread block per (group, token).
__global__ __launch_bounds__(256) void k_pf_swiglu_quant(const float* __restrict__ gu, int I, int gs, float gscale,
                                                         int8_t* __restrict__ xq, float* __restrict__ xs) {
    const int g = blockIdx.x, tok = blockIdx.y, t = threadIdx.x, ng = I / gs;
    __shared__ float red[4];
    const float* row = gu + (size_t)tok * 2 * I;
    auto value = [&](int i) __attribute__((always_inline)) {
        const int gr = (i >> 4) * 32 + (i & 15);
        const float gv = row[gr], uv = row[gr + 16];
        const float swv = gv / (1.0f + qexp(-gv));
        return swv * uv * gscale;
    };
    constexpr int VPT = 8;                         // values per thread held for the two passes
    float v[VPT];
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const int i = g * gs + t + 256 * u;
        v[u] = 0.0f;
        if (t + 256 * u < gs) {
            v[u] = value(i);
            mx = fmaxf(mx, fabsf(v[u]));
        }
    }
    mx = max_xor(mx, 64);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = m * (1.0f / 127.0f), qi = (sc > 0.0f) ? 1.0f / sc : 0.0f;
    if (t == 0) xs[(size_t)tok * ng + g] = sc;
#pragma unroll
    for (int u = 0; u < VPT; ++u)
        if (t + 256 * u < gs) xq[(size_t)tok * I + g * gs + t + 256 * u] = qcode(v[u], qi);
}
// The same for groups wider than 2048 outputs (the whole I, the default arm): one 1024-thread
// block per (group, token) holds the group's values in registers, four consecutive outputs per
// thread and chunk (one 16-byte gate and one 16-byte up load, one 4-byte code store), so every
// value is computed once; the max, scale and codes are those of the kernel above.
constexpr int kSwWideT = 1024, kSwWideQ = 5;       // threads, quads per thread (gs <= 20480)
__global__ __launch_bounds__(kSwWideT) void k_pf_swiglu_quant_wide(const float* __restrict__ gu, int I, int gs,
                                                                  float gscale, int8_t* __restrict__ xq,
                                                                  float* __restrict__ xs) {
    const int g = blockIdx.x, tok = blockIdx.y, t = threadIdx.x, ng = I / gs;
    __shared__ float red[kSwWideT / 64];
    const float* row = gu + (size_t)tok * 2 * I;
    float v[kSwWideQ][4];
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < kSwWideQ; ++u) {
        const int j = 4 * (t + kSwWideT * u);      // output within the group
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = 0.0f;
        if (j < gs) {
            const int i = g * gs + j, gr = (i >> 4) * 32 + (i & 15);
            const float4 gv4 = *(const float4*)(row + gr), uv4 = *(const float4*)(row + gr + 16);
            const float gv[4] = {gv4.x, gv4.y, gv4.z, gv4.w}, uv[4] = {uv4.x, uv4.y, uv4.z, uv4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float swv = gv[e] / (1.0f + qexp(-gv[e]));
                v[u][e] = swv * uv[e] * gscale;
                mx = fmaxf(mx, fabsf(v[u][e]));
            }
        }
    }
    mx = max_xor(mx, 64);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < kSwWideT / 64; ++w) m = fmaxf(m, red[w]);
    const float sc = m * (1.0f / 127.0f), qi = (sc > 0.0f) ? 1.0f / sc : 0.0f;
    if (t == 0) xs[(size_t)tok * ng + g] = sc;
#pragma unroll
    for (int u = 0; u < kSwWideQ; ++u) {
        const int j = 4 * (t + kSwWideT * u);
        if (j < gs) {
            uint32_t pk = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) pk |= ((uint32_t)(uint8_t)qcode(v[u][e], qi)) << (8 * e);
            *(uint32_t*)(xq + (size_t)tok * I + (size_t)g * gs + j) = pk;
        }
    }
}
int launch_pf_swiglu_quant(const float* gu, int I, int gs, float gscale, int C, int8_t* xq, float* xs,
                           hipStream_t s) {
    if (!gu || !xq || !xs || C < 1 || (I & 31) || gs < 16 || (gs & 15) || (I % gs) || gs > 4 * kSwWideT * kSwWideQ ||
        ((uintptr_t)gu & 15) || ((uintptr_t)xq & 3) || (I & 3)) {
        set_error("prefill swiglu: bad arguments (I %d, gs %d)", I, gs);
        return Q27X_E_ARG;
    }
    if (gs > 256 * 8)
        hipLaunchKernelGGL(k_pf_swiglu_quant_wide, dim3((unsigned)(I / gs), (unsigned)C), dim3(kSwWideT), 0, s, gu, I, gs,
                           gscale, xq, xs);
    else
        hipLaunchKernelGGL(k_pf_swiglu_quant, dim3((unsigned)(I / gs), (unsigned)C), dim3(256), 0, s, gu, I, gs, gscale,
                           xq, xs);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

}  // namespace q27x
