// k_gemm.hip -- prefill ingest on int8 MFMA: the per-(row, group) W8A8 GEMM of the reference's
// layer-split prefill and its two quantizers, as hand-written gfx950 kernels.
//
// Reference: one rocBLAS int8 gemm_ex per K group writes an int32 slab (src/q27_rb.cpp:43-55), and
// an epilogue sums the slabs with the product of the two scales (src/q27_epi.hip:189-203, fp32 +
// residual form 235-243). The groups are GS = 1024 columns (or the whole K); weights are the
// per-64 mirror requantized per (row, group) (src/q27_epi.hip:14-35), activations are quantized
// per (token, group) (q27_quant_group, src/q27_epi.hip:64-75).
//
// Semantics kept bit for bit:
//   weights:     sg = max of the group's per-64 scales; inv = sg > 0 ? 1/sg : 0;
//                code = clamp(rint(((float)w * s64) * inv), -127, 127)
//   activations: sc = max|v| * (1/127); qi = sc > 0 ? 1/sc : 0; code = clamp(rint(v * qi), -127, 127)
//   GEMM:        acc_g = exact int32 dot over group g; o = 0;
//                for g ascending: o = fmaf((float)acc_g, sw[n][g] * sx[t][g], o);
//                y[t][n] = o * alpha (+ rs * res[t][n])
// The int32 group sums do not depend on the order of their terms, so the MFMA tiling cannot
// change them; the fp32 part runs per output in the reference's group order.
//
// GEMM tiling: a 256-thread block computes a 128-token x 128-row tile; wave w owns the 64 x 64
// quarter (w / 2, w % 2) as 2 x 2 v_mfma_i32_32x32x32_i8 tiles. K advances 128 bytes per step
// through a double-buffered LDS stage whose rows are padded to 144 bytes, so the 32 rows that
// one operand read touches start in distinct banks. The next step's tiles are loaded into
// registers while the current step is multiplied. At the end of each group the int32 tiles are
// folded into fp32 accumulators with the group's scales (staged in LDS for the whole K at the
// start) and restarted from zero.
#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kGM = 128, kGN = 128, kGK = 128;    // block tile: tokens x weight rows x K bytes
constexpr int kGLd = kGK + 16;                     // LDS row pitch (bytes)
constexpr int kGMaxG = 20;                         // groups per row held in LDS (K / GS)

struct GemmArgs {
    const int8_t* w;    // [N][K] per-(row, group) codes
    const float* sw;    // [N][ng]
    const int8_t* x;    // [M][K] per-(token, group) codes
    const float* sx;    // [M][ng]
    float* y;           // [M][ldy]
    const float* res;   // [M][ldr] or null
    float alpha, rs;
    int M, N, K, gs, ng, ldy, ldr;
};

__global__ __launch_bounds__(256) void k_gemm_i8g(GemmArgs a) {
    __shared__ __align__(16) int8_t sA[2][kGM * kGLd];
    __shared__ __align__(16) int8_t sB[2][kGN * kGLd];
    __shared__ float sSx[kGM * kGMaxG];
    __shared__ float sSw[kGN * kGMaxG];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * kGN, m0 = blockIdx.y * kGM;
    const int K = a.K, ng = a.ng, spg = a.gs / kGK, nsteps = K / kGK;

    // the block's scales for every group (rows past M read row M - 1; their outputs are not stored)
    for (int i = tid; i < kGM * ng; i += 256) {
        const int r = i / ng, g = i - r * ng;
        const int t = (m0 + r < a.M) ? m0 + r : a.M - 1;
        sSx[r * kGMaxG + g] = a.sx[(size_t)t * ng + g];
        sSw[r * kGMaxG + g] = a.sw[(size_t)(n0 + r) * ng + g];
    }

    // register stage: thread tid moves the 16-byte chunks c = tid + 256 q (q < 4) of each tile,
    // chunk c = row c / 8, bytes 16 (c % 8) .. +16 of the step (8 threads cover one 128-byte row).
    // (Plain code rather than lambdas: captured arrays were moved to LDS by the compiler.)
    const int crow = tid >> 3, ccol = (tid & 7) * 16;
    const int8_t* xp[4];
    const int8_t* wp[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int row = crow + 32 * q;
        const int t = (m0 + row < a.M) ? m0 + row : a.M - 1;
        xp[q] = a.x + (size_t)t * K + ccol;
        wp[q] = a.w + (size_t)(n0 + row) * K + ccol;
    }
    uint4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
#define Q27X_GLOAD(k0)                                                                              \
    ra0 = *(const uint4*)(xp[0] + (k0)); rb0 = *(const uint4*)(wp[0] + (k0));                       \
    ra1 = *(const uint4*)(xp[1] + (k0)); rb1 = *(const uint4*)(wp[1] + (k0));                       \
    ra2 = *(const uint4*)(xp[2] + (k0)); rb2 = *(const uint4*)(wp[2] + (k0));                       \
    ra3 = *(const uint4*)(xp[3] + (k0)); rb3 = *(const uint4*)(wp[3] + (k0));
#define Q27X_SSTORE(buf)                                                                            \
    *(uint4*)&sA[buf][(crow) * kGLd + ccol] = ra0; *(uint4*)&sB[buf][(crow) * kGLd + ccol] = rb0;   \
    *(uint4*)&sA[buf][(crow + 32) * kGLd + ccol] = ra1; *(uint4*)&sB[buf][(crow + 32) * kGLd + ccol] = rb1; \
    *(uint4*)&sA[buf][(crow + 64) * kGLd + ccol] = ra2; *(uint4*)&sB[buf][(crow + 64) * kGLd + ccol] = rb2; \
    *(uint4*)&sA[buf][(crow + 96) * kGLd + ccol] = ra3; *(uint4*)&sB[buf][(crow + 96) * kGLd + ccol] = rb3;

    v16i acc[2][2];
    float facc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) { acc[i][j][r] = 0; facc[i][j][r] = 0.0f; }

    // operand rows of this lane: A row (token) wm*64 + 32 i + lane % 32, B row (weight row)
    // wn*64 + 32 j + lane % 32; both take bytes 16 (lane / 32) .. +16 of each 32-byte K slice, so
    // A and B pair the same K positions
    const int arow = wm * 64 + (lane & 31), brow = wn * 64 + (lane & 31), kh = (lane >> 5) * 16;

    Q27X_GLOAD(0)
    Q27X_SSTORE(0)
    __syncthreads();
    for (int s = 0; s < nsteps; ++s) {
        const int buf = s & 1;
        // the step after the last reloads step 0 into the idle buffer (nothing reads it), so
        // every iteration issues the same loads and the compiler's waits stay exact
        const int kn = (s + 1 < nsteps ? s + 1 : 0) * kGK;
        Q27X_GLOAD(kn)
#pragma unroll
        for (int kk = 0; kk < kGK / 32; ++kk) {
            v4i av0 = *(const v4i*)&sA[buf][arow * kGLd + kk * 32 + kh];
            v4i av1 = *(const v4i*)&sA[buf][(arow + 32) * kGLd + kk * 32 + kh];
            v4i bv0 = *(const v4i*)&sB[buf][brow * kGLd + kk * 32 + kh];
            v4i bv1 = *(const v4i*)&sB[buf][(brow + 32) * kGLd + kk * 32 + kh];
            acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av0, bv0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av0, bv1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av1, bv0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av1, bv1, acc[1][1], 0, 0, 0);
        }
        if ((s + 1) % spg == 0) {
            // fold the group: accumulator element r of a 32 x 32 tile is row
            // 8 (r / 4) + 4 (lane / 32) + r % 4, column lane % 32
            const int g = (s + 1) / spg - 1;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float swv = sSw[(brow + 32 * j) * kGMaxG + g];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int tr = wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        const float sc = swv * sSx[tr * kGMaxG + g];
                        facc[i][j][r] = __builtin_fmaf((float)acc[i][j][r], sc, facc[i][j][r]);
                        acc[i][j][r] = 0;
                    }
            }
        }
        Q27X_SSTORE(buf ^ 1)
        __syncthreads();
    }
#undef Q27X_GLOAD
#undef Q27X_SSTORE

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = n0 + wn * 64 + 32 * j + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int t = m0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (t < a.M) {
                    float o = facc[i][j][r] * a.alpha;
                    if (a.res) o = o + a.rs * a.res[(size_t)t * a.ldr + n];
                    a.y[(size_t)t * a.ldy + n] = o;
                }
            }
        }
}

// Weights: per-64 mirror -> per-(row, group) codes and scales; one 256-thread block per row.
// In place when wg == w (each element is read and written by the same thread).
__global__ __launch_bounds__(256) void k_i8g64_to_grp(const int8_t* w, const float* s64, int K, int gs,
                                                      int8_t* wg, float* sg) {
    const int r = blockIdx.x, t = threadIdx.x, ns = K >> 6, ng = K / gs;
    __shared__ float red[4];
    const int8_t* row = w + (size_t)r * K;
    int8_t* out = wg + (size_t)r * K;
    const float* sr = s64 + (size_t)r * ns;
    for (int g = 0; g < ng; ++g) {
        float mx = 0.0f;
        for (int i = t; i < (gs >> 6); i += 256) mx = fmaxf(mx, sr[g * (gs >> 6) + i]);
        mx = max_xor(mx, 64);
        if ((t & 63) == 0) red[t >> 6] = mx;
        __syncthreads();
        const float s = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        const float inv = (s > 0.0f) ? 1.0f / s : 0.0f;
        if (t == 0) sg[(size_t)r * ng + g] = s;
        for (int k = g * gs + t; k < (g + 1) * gs; k += 256) {
            out[k] = qcode((float)row[k] * sr[k >> 6], inv);
        }
    }
}

// Activations: fp32 rows -> per-(token, group) codes and scales; one 256-thread block per
// (group, token), four values per thread per 1024 columns.
__global__ __launch_bounds__(256) void k_quant_tok_grp(const float* x, int xstride, int K, int gs, int8_t* xq,
                                                       float* xs) {
    const int g = blockIdx.x, tok = blockIdx.y, t = threadIdx.x, ng = K / gs;
    __shared__ float red[4];
    const float* row = x + (size_t)tok * xstride + (size_t)g * gs;
    float mx = 0.0f;
    for (int k = 4 * t; k < gs; k += 1024) {
        const float4 v = *(const float4*)(row + k);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    mx = max_xor(mx, 64);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = m * (1.0f / 127.0f), qi = (sc > 0.0f) ? 1.0f / sc : 0.0f;
    if (t == 0) xs[(size_t)tok * ng + g] = sc;
    int8_t* out = xq + (size_t)tok * K + (size_t)g * gs;
    for (int k = 4 * t; k < gs; k += 1024) {
        const float4 v = *(const float4*)(row + k);
        const uint32_t pk = (uint32_t)(uint8_t)qcode(v.x, qi) | ((uint32_t)(uint8_t)qcode(v.y, qi) << 8) |
                            ((uint32_t)(uint8_t)qcode(v.z, qi) << 16) | ((uint32_t)(uint8_t)qcode(v.w, qi) << 24);
        *(uint32_t*)(out + k) = pk;
    }
}

}  // namespace q27x

// ---------------------------------------------------------------- C ABI (prefill GEMM tier)
using namespace q27x;

extern "C" int q27x_i8g64_to_grp(const int8_t* w, const float* s64, int rows, int K, int gs, int8_t* wg,
                                 float* sg, q27x_stream_t s) {
    if (!w || !s64 || !wg || !sg || rows < 1 || K < 64 || gs < 64 || (gs & 63) || (K % gs)) {
        set_error("q27x_i8g64_to_grp: bad arguments (rows %d, K %d, gs %d)", rows, K, gs);
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_i8g64_to_grp, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)s, w, s64, K, gs, wg, sg);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

extern "C" int q27x_quant_tok_groups(const float* x, int xstride, int M, int K, int gs, int8_t* xq, float* xs,
                                     q27x_stream_t s) {
    if (!x || !xq || !xs || M < 1 || K < 4 || gs < 4 || (gs & 3) || (K % gs) || xstride < K || (xstride & 3) ||
        ((uintptr_t)x & 15)) {
        set_error("q27x_quant_tok_groups: bad arguments (M %d, K %d, gs %d, xstride %d)", M, K, gs, xstride);
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_quant_tok_grp, dim3((unsigned)(K / gs), (unsigned)M), dim3(256), 0, (hipStream_t)s, x,
                       xstride, K, gs, xq, xs);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

extern "C" int q27x_gemm_i8g(const int8_t* w, const float* sw, int N, int K, int gs, float alpha, const int8_t* x,
                             const float* sx, int M, float* y, int ldy, const float* res, int ldr, float rs,
                             q27x_stream_t s) {
    if (!w || !sw || !x || !sx || !y || M < 1 || N < 1 || K < 1 || gs < 1 || ldy < N || (res && ldr < N)) {
        set_error("q27x_gemm_i8g: bad arguments");
        return Q27X_E_ARG;
    }
    if ((N % kGN) || (K % kGK) || (gs % kGK) || (K % gs) || K / gs > kGMaxG || ((uintptr_t)w & 15) ||
        ((uintptr_t)x & 15)) {
        set_error("q27x_gemm_i8g: no kernel for N %d, K %d, gs %d (N %% %d, K %% %d, gs %% %d must be 0, "
                  "K/gs <= %d, 16-byte aligned codes)", N, K, gs, kGN, kGK, kGK, kGMaxG);
        return Q27X_E_SHAPE;
    }
    GemmArgs a{};
    a.w = w; a.sw = sw; a.x = x; a.sx = sx; a.y = y; a.res = res; a.alpha = alpha; a.rs = rs;
    a.M = M; a.N = N; a.K = K; a.gs = gs; a.ng = K / gs; a.ldy = ldy; a.ldr = ldr;
    hipLaunchKernelGGL(k_gemm_i8g, dim3((unsigned)(N / kGN), (unsigned)((M + kGM - 1) / kGM)), dim3(256), 0,
                       (hipStream_t)s, a);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
