// k_gdn.hip -- gated-delta-rule verify of NR rows with deferred commit (R10-R12).
//
// Mathematics (src/q27_gdn.hip:206-372, gdn_step_body), per value head h, key head h/ratio:
//   q^ = q rsqrt(sum q^2 + 1e-6) / sqrt(128), k^ = k rsqrt(sum k^2 + 1e-6)
//   beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a + dt_bias))
//   A = S^T k^, B = S^T q^, delta = (v - decay A) beta, mixed = decay B + delta (k^.q^)
//   S <- decay S + k^ (x) delta
//   out = mixed rsqrt(mean(mixed^2) + eps) norm_w SiLU(z)  -> bf16 -> per-16 int8
// Layout: S [VH][D=128][D] fp32 key-major. Four blocks per head, each owning 32 value dims of
// all 128 key rows (16 KiB of state, 32 floats per thread, VGPR-resident for every row of the
// verify); the four blocks of a head are placed on one XCD so they share an L2.
// Rollback: instead of the reference's per-row snapshot banks (src/q27_main.cpp:2933-2941) the
// state in HBM stays at the last committed position; each row's (k^, delta, decay) goes to
// `pend`, and the next call first applies the rows that were accepted (npend), writes that state
// back once, then continues. The commit uses exactly the update the row already received, so the
// committed state is bit-identical to stepping the accepted rows one at a time.
#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

constexpr int kD = 128;
constexpr int kDSplit = 4;            // blocks per value head
constexpr int kDB = kD / kDSplit;     // value dims per block (32)
constexpr int kNT = 4 * kDB;          // threads: 4 key groups x 32 value dims
constexpr int kJ = kD / 4;            // key rows per thread (32)

// pend buffer: header (parity, global counter, per-head counters) | two parity areas of
// khat [R][KH][D] | delta [R][VH][D] | decay [R][VH] | mixed [R][VH][D] | raw [R][NQKV] bf16 |
// work [R][NQKV] bf16 (conv output of the kernel-tier entry). A call reads the pending rows from
// area `par` and writes its own rows to area 1-par; the last block of the grid flips par, so no
// block can overwrite a vector a sibling block has still to read.
__host__ __device__ static inline size_t hdr_bytes(int vh) { return (((size_t)(2 + vh) * 4) + 255) & ~(size_t)255; }
__host__ __device__ static inline size_t area_floats(int kh, int vh) {
    return (size_t)kMaxRows * ((size_t)kh * kD + (size_t)vh * kD + vh);
}
size_t gdn_pend_raw_offset(int kh, int vh, int d) {
    (void)d;
    return hdr_bytes(vh) + (2 * area_floats(kh, vh) + (size_t)kMaxRows * vh * kD) * 4;
}
size_t gdn_pend_bytes(int kh, int vh, int d) {
    const size_t nqkv = (size_t)(2 * kh + vh) * d;
    return gdn_pend_raw_offset(kh, vh, d) + 2 * (size_t)kMaxRows * nqkv * 2;
}
struct PendHdr { unsigned par; unsigned gcnt; unsigned hcnt[1]; };
struct PendArea { float* khat; float* delta; float* decay; };
__device__ __forceinline__ PendArea pend_area(void* p, int kh, int vh, int which) {
    float* b = (float*)((char*)p + hdr_bytes(vh)) + (size_t)which * area_floats(kh, vh);
    PendArea v;
    v.khat = b;  b += (size_t)kMaxRows * kh * kD;
    v.delta = b; b += (size_t)kMaxRows * vh * kD;
    v.decay = b;
    return v;
}
__device__ __forceinline__ float* pend_mixed(void* p, int kh, int vh) {
    return (float*)((char*)p + hdr_bytes(vh)) + 2 * area_floats(kh, vh);
}

template <int FUSE_AB>
__global__ __launch_bounds__(kNT) void k_gdn(GdnArgs a, int nr) {
    if (a.stop && *a.stop) return;
    // XCD-aware placement: block b runs on XCD b%8; the 4 blocks of a head share one XCD.
    const int nb = gridDim.x;                       // vh * 4
    const int b = blockIdx.x;
    int h, dq;
    if ((nb & 7) == 0 && ((nb >> 3) % kDSplit) == 0) {
        const int x = b & 7, i = b >> 3;            // XCD, index within the XCD
        const int hx = (nb >> 3) / kDSplit;         // heads per XCD
        h = x * hx + i / kDSplit;
        dq = i % kDSplit;
    } else { h = b / kDSplit; dq = b % kDSplit; }
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int dl = t & (kDB - 1), g = t / kDB;      // local value dim, key group
    const int d = dq * kDB + dl;
    const int ratio = a.vh / a.kh, kk = h / ratio;
    const int KD = a.kh * kD;
    PendHdr* hdr = (PendHdr*)a.pend;
    const unsigned par = hdr->par & 1u;
    const PendArea P = pend_area(a.pend, a.kh, a.vh, (int)par);       // pending rows (read)
    const PendArea Q = pend_area(a.pend, a.kh, a.vh, (int)(par ^ 1u)); // this call's rows (write)
    float* mixed_g = pend_mixed(a.pend, a.kh, a.vh);
    __shared__ float sq[kD], sk[kD];
    __shared__ float pA[4][kDB], pB[4][kDB];
    __shared__ float red[2][3];
    __shared__ float sab[2][kMaxRows];
    __shared__ float skp[kMaxRows][kD];
    __shared__ float sdp[kMaxRows][kDB];
    __shared__ float sdc[kMaxRows];
    __shared__ unsigned s_last;
    const int npend = a.npend_ptr ? *a.npend_ptr : a.npend_imm;

    // ---- a / b logits: bf16 GEMV of in_a / in_b row h on the bf16 normed rows (lane-chunk
    //      order; bf16 rounding of the result as k_bf16_gemv2_tile, src/q27_util.hip:158-162)
    if (FUSE_AB) {
        for (int q = wv; q < 2 * nr; q += kNT / 64) {
            const int which = q & 1, n = q >> 1;
            const uint16_t* wr = (which ? a.in_b : a.in_a) + (size_t)h * a.H;
            const uint16_t* yr = a.ynorm + (size_t)n * a.ystride;
            float acc = 0.0f;
            for (int c = lane; c < (a.H >> 3); c += 64) {
                const uint4 w = *(const uint4*)(wr + 8 * c);
                const uint4 y = *(const uint4*)(yr + 8 * c);
                acc = __builtin_fmaf(__uint_as_float(w.x << 16), __uint_as_float(y.x << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w.x & 0xFFFF0000u), __uint_as_float(y.x & 0xFFFF0000u), acc);
                acc = __builtin_fmaf(__uint_as_float(w.y << 16), __uint_as_float(y.y << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w.y & 0xFFFF0000u), __uint_as_float(y.y & 0xFFFF0000u), acc);
                acc = __builtin_fmaf(__uint_as_float(w.z << 16), __uint_as_float(y.z << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w.z & 0xFFFF0000u), __uint_as_float(y.z & 0xFFFF0000u), acc);
                acc = __builtin_fmaf(__uint_as_float(w.w << 16), __uint_as_float(y.w << 16), acc);
                acc = __builtin_fmaf(__uint_as_float(w.w & 0xFFFF0000u), __uint_as_float(y.w & 0xFFFF0000u), acc);
            }
            acc = tree64(acc);
            if (lane == 0) sab[which][n] = bfr(acc);
        }
    } else if (t < 2 * nr) {
        const int which = t & 1, n = t >> 1;
        sab[which][n] = (which ? a.b : a.a)[(size_t)n * a.ab_stride + h];
    }

    // ---- the committed state of this block's slice, plus the pending rows
    float* Sp = a.S + (size_t)h * kD * kD + (size_t)(g * kJ) * kD + d;
    float st[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) st[j] = Sp[(size_t)j * kD];
    for (int i = t; i < npend * kD; i += kNT) {
        const int p = i / kD, j = i - p * kD;
        skp[p][j] = P.khat[((size_t)p * a.kh + kk) * kD + j];
    }
    for (int i = t; i < npend * kDB; i += kNT) {
        const int p = i / kDB, e = i - p * kDB;
        sdp[p][e] = P.delta[((size_t)p * a.vh + h) * kD + dq * kDB + e];
    }
    if (t < npend) sdc[t] = P.decay[(size_t)t * a.vh + h];
    __syncthreads();
    for (int p = 0; p < npend; ++p) {
        const float dp = sdp[p][dl], dc = sdc[p];
#pragma unroll
        for (int j = 0; j < kJ; ++j) st[j] = __builtin_fmaf(skp[p][g * kJ + j], dp, dc * st[j]);
    }
    if (npend > 0) {
#pragma unroll
        for (int j = 0; j < kJ; ++j) Sp[(size_t)j * kD] = st[j];
    }

    const float Aexp = qexp(bf2f(a.A_log[h]));
    const float dtb = bf2f(a.dt_bias[h]);
    for (int n = 0; n < nr; ++n) {
        const uint16_t* row = a.qkv + (size_t)n * a.qkv_stride;
        // q/k L2 norms and k^.q^: two waves, one element per lane (redundant in every block)
        {
            const float qv = bf2f(row[kk * kD + t]);
            const float kv = bf2f(row[KD + kk * kD + t]);
            const float r0 = tree64(qv * qv), r1 = tree64(kv * kv), r2 = tree64(qv * kv);
            if (lane == 0) { red[wv][0] = r0; red[wv][1] = r1; red[wv][2] = r2; }
        }
        __syncthreads();
        const float sumq2 = red[0][0] + red[1][0];
        const float sumk2 = red[0][1] + red[1][1];
        const float sumqk = red[0][2] + red[1][2];
        const float invq = rsqrt_cr(sumq2 + 1e-6f) * 0.0883883476f;
        const float invk = rsqrt_cr(sumk2 + 1e-6f);
        const float kq = sumqk * invq * invk;
        sq[t] = bf2f(row[kk * kD + t]) * invq;
        sk[t] = bf2f(row[KD + kk * kD + t]) * invk;
        const float beta = qsigmoid(sab[1][n]);
        const float sp = qsoftplus(sab[0][n] + dtb);
        const float decay = qexp(-(Aexp * sp));
        const float vv = bf2f(row[2 * KD + h * kD + d]);
        __syncthreads();
        float accA = 0.0f, accB = 0.0f;
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
            accA = __builtin_fmaf(st[j], sk[g * kJ + j], accA);
            accB = __builtin_fmaf(st[j], sq[g * kJ + j], accB);
        }
        pA[g][dl] = accA;
        pB[g][dl] = accB;
        __syncthreads();
        const float A = ((pA[0][dl] + pA[1][dl]) + pA[2][dl]) + pA[3][dl];
        const float B = ((pB[0][dl] + pB[1][dl]) + pB[2][dl]) + pB[3][dl];
        const float delta = (vv - decay * A) * beta;
        const float mixed = __builtin_fmaf(delta, kq, decay * B);
#pragma unroll
        for (int j = 0; j < kJ; ++j) st[j] = __builtin_fmaf(sk[g * kJ + j], delta, decay * st[j]);
        if (g == 0) {
            Q.delta[((size_t)n * a.vh + h) * kD + d] = delta;
            mixed_g[((size_t)n * a.vh + h) * kD + d] = mixed;
        }
        if (dq == 0 && t == 0) Q.decay[(size_t)n * a.vh + h] = decay;
        if (dq == 0 && (h % ratio) == 0) Q.khat[((size_t)n * a.kh + kk) * kD + t] = sk[t];
        __syncthreads();   // sq / sk / red reused by the next row
    }

    // ---- output norm + gate + quantize: the last of the head's four blocks does all rows
    __threadfence();
    __syncthreads();
    if (t == 0) s_last = (atomicAdd(&hdr->hcnt[h], 1u) == (unsigned)(kDSplit - 1)) ? 1u : 0u;
    __syncthreads();
    if (s_last) {
        __threadfence();
        const float nw = bf2f(a.norm_w[t]);
        for (int n = 0; n < nr; ++n) {
            const float mx = __builtin_nontemporal_load(&mixed_g[((size_t)n * a.vh + h) * kD + t]);
            const float r3 = tree64(mx * mx);
            if (lane == 0) red[wv][0] = r3;
            __syncthreads();
            const float summ = red[0][0] + red[1][0];
            const float inv = rsqrt_cr(summ * (1.0f / (float)kD) + a.eps);
            const float z = bf2f(a.z[(size_t)n * a.z_stride + (size_t)h * kD + t]);
            const float y = mx * inv * nw * qsilu(z);
            const uint16_t yb = f2bf(y);
            a.out[(size_t)n * a.out_stride + (size_t)h * kD + t] = yb;
            if (a.xq) {
                const float yv = bf2f(yb);
                const float m16 = max_xor(fabsf(yv), 16);
                const float sc = m16 * (1.0f / 127.0f);
                const float qi = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
                const size_t k = (size_t)n * a.out_stride + (size_t)h * kD + t;
                a.xq[k] = qcode(yv, qi);
                if ((t & 15) == 0) a.xs[k >> 4] = sc;
            }
            __syncthreads();
        }
        if (t == 0) hdr->hcnt[h] = 0u;
    }
    // ---- the last block of the grid flips the parity (every block has read it by now)
    if (t == 0) {
        __threadfence();
        if (atomicAdd(&hdr->gcnt, 1u) == (unsigned)(nb - 1)) {
            hdr->gcnt = 0u;
            hdr->par = par ^ 1u;
            __threadfence();
        }
    }
}

int launch_gdn(const GdnArgs& a, int nr, hipStream_t s) {
    if (a.d != kD || a.kh < 1 || a.vh % a.kh || nr < 1 || nr > kMaxRows || !a.qkv || !a.z || !a.S || !a.pend || !a.out) {
        set_error("gdn: unsupported shape or null argument (d=%d kh=%d vh=%d nr=%d)", a.d, a.kh, a.vh, nr);
        return Q27X_E_SHAPE;
    }
    if (a.xq && a.out_stride % 16) { set_error("gdn: out_stride must be a multiple of 16"); return Q27X_E_ARG; }
    const int fuse = (a.in_a && a.in_b && a.ynorm) ? 1 : 0;
    if (!fuse && (!a.a || !a.b)) { set_error("gdn: a/b logits or in_a/in_b weights required"); return Q27X_E_ARG; }
    const int grid = a.vh * kDSplit;
    if (fuse) hipLaunchKernelGGL(k_gdn<1>, dim3(grid), dim3(kNT), 0, s, a, nr);
    else hipLaunchKernelGGL(k_gdn<0>, dim3(grid), dim3(kNT), 0, s, a, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// conv + SiLU with the deferred shift-register commit as a standalone kernel (the engine fuses
// it into the in_qkv projection epilogue; this form serves the kernel-tier entry and its tests)
__global__ __launch_bounds__(256) void k_gdn_conv(const uint16_t* __restrict__ raw, int raw_stride,
                                                  uint16_t* __restrict__ out, int out_stride, int nconv,
                                                  const uint16_t* __restrict__ conv_w, uint16_t* __restrict__ hist,
                                                  uint16_t* __restrict__ pend_raw, const int* npend_ptr, int npend_imm,
                                                  int nr) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= nconv) return;
    const int npend = npend_ptr ? *npend_ptr : npend_imm;
    uint16_t h0 = hist[3 * c], h1 = hist[3 * c + 1], h2 = hist[3 * c + 2];
    for (int p = 0; p < npend; ++p) { h0 = h1; h1 = h2; h2 = pend_raw[(size_t)p * nconv + c]; }
    hist[3 * c] = h0; hist[3 * c + 1] = h1; hist[3 * c + 2] = h2;
    const float w0 = bf2f(conv_w[4 * c]), w1 = bf2f(conv_w[4 * c + 1]);
    const float w2 = bf2f(conv_w[4 * c + 2]), w3 = bf2f(conv_w[4 * c + 3]);
    for (int n = 0; n < nr; ++n) {
        const uint16_t x = raw[(size_t)n * raw_stride + c];
        float acc = bf2f(h0) * w0;
        acc = __builtin_fmaf(bf2f(h1), w1, acc);
        acc = __builtin_fmaf(bf2f(h2), w2, acc);
        acc = __builtin_fmaf(bf2f(x), w3, acc);
        h0 = h1; h1 = h2; h2 = x;
        pend_raw[(size_t)n * nconv + c] = x;
        out[(size_t)n * out_stride + c] = f2bf(qsilu(acc));
    }
}
int launch_gdn_conv(const uint16_t* raw, int raw_stride, uint16_t* out, int out_stride, int nconv,
                    const uint16_t* conv_w, uint16_t* conv_hist, uint16_t* pend_raw, const int* npend_ptr,
                    int npend_imm, int nr, hipStream_t s) {
    hipLaunchKernelGGL(k_gdn_conv, dim3((nconv + 255) / 256), dim3(256), 0, s, raw, raw_stride, out, out_stride,
                       nconv, conv_w, conv_hist, pend_raw, npend_ptr, npend_imm, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

}  // namespace q27x

using namespace q27x;
extern "C" size_t q27x_gdn_pend_bytes(int kh, int vh, int d, int max_rows) {
    (void)max_rows;
    return gdn_pend_bytes(kh, vh, d);
}

// Kernel-tier entry: conv (deferred commit) then the recurrence. The conv'd rows go to the work
// area at the end of `pend`, so the call allocates nothing.
extern "C" int q27x_gdn_verify(const uint16_t* qkv_raw, int qkv_stride, const uint16_t* z, int z_stride,
                               const float* a, const float* b, int ab_stride, const uint16_t* A_log,
                               const uint16_t* dt_bias, const uint16_t* norm_w, const uint16_t* conv_w, float* S,
                               uint16_t* conv_hist, void* pend, int npend, int kh, int vh, int d, uint16_t* out,
                               int out_stride, int8_t* xq, float* xs, int nr, q27x_stream_t s) {
    if (!qkv_raw || !z || !a || !b || !S || !conv_hist || !pend || !out || nr < 1 || nr > kMaxRows ||
        npend < 0 || npend > kMaxRows || d != 128) {
        set_error("q27x_gdn_verify: bad arguments");
        return Q27X_E_ARG;
    }
    const int nconv = (2 * kh + vh) * d;
    uint16_t* pend_raw = (uint16_t*)((char*)pend + gdn_pend_raw_offset(kh, vh, d));
    uint16_t* conv_buf = pend_raw + (size_t)kMaxRows * nconv;
    int rc = launch_gdn_conv(qkv_raw, qkv_stride, conv_buf, nconv, nconv, conv_w, conv_hist, pend_raw, nullptr,
                             npend, nr, (hipStream_t)s);
    if (rc) return rc;
    GdnArgs g{};
    g.qkv = conv_buf; g.qkv_stride = nconv; g.z = z; g.z_stride = z_stride;
    g.a = a; g.b = b; g.ab_stride = ab_stride;
    g.A_log = A_log; g.dt_bias = dt_bias; g.norm_w = norm_w; g.S = S; g.pend = pend;
    g.npend_imm = npend; g.kh = kh; g.vh = vh; g.d = d; g.eps = 1e-6f;
    g.out = out; g.out_stride = out_stride; g.xq = xq; g.xs = xs;
    return launch_gdn(g, nr, (hipStream_t)s);
}
