// k_gdn.hip -- gated-delta-rule verify of NR rows with deferred commit (R10-R12).
//
// Mathematics (src/q27_gdn.hip:206-372, gdn_step_body; the NR scan k_gdn_scan_tp, 464-592), per
// value head h, key head h/ratio:
//   q^ = q rsqrt(sum q^2 + 1e-6) / sqrt(128), k^ = k rsqrt(sum k^2 + 1e-6)
//   beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a + dt_bias))
//   A = S^T k^, B = S^T q^, delta = (v - decay A) beta, mixed = decay B + delta (k^.q^)
//   S <- decay S + k^ (x) delta            (row by row, as the reference's scan)
//   out = mixed rsqrt(mean(mixed^2) + eps) norm_w SiLU(z)  -> bf16 -> per-16 int8
// Layout: S [VH][D=128][D] fp32 key-major. One 512-thread block per value head: thread (g, d)
// holds key rows 32g..32g+31 of value column d (64 KiB of state per block in VGPRs). Every
// global load of the block is issued before the first wait, so a call costs one memory round
// trip plus on-chip work; the rows then run with one barrier each. A head stays on one block: the
// output norm sums mixed^2 over all 128 value columns, so a head split over two blocks (columns
// 0..63 | 64..127, the prefill scan's lane layout, no barrier per row) has to exchange the two
// halves' sums; with agent-scope stores, an arrival counter and the second block finishing the
// head, that form was bit-exact but measured 12.4 us against this kernel's 8.5 us at 3 rows
// (10.36 against 10.20 ms per K=7 round), the exchange's dependent round trips costing more than
// the halved work per SIMD saves.
// Inputs arrive prepared: the engine convolves the q|k|v channels in the epilogue of the
// in_qkv|in_z projection and computes each row's (decay, beta) there as well (the a/b dot products
// and their transcendentals, k_proj), so `rowsc` holds them; the kernel-tier entry passes the a/b
// logits instead (the scalars are then computed here) and convolves with k_gdn_conv first.
// Rollback: instead of the reference's per-row snapshot banks (src/q27_main.cpp:2933-2941) the
// state in HBM stays at the last committed position; each row's (k^, delta, decay) goes to
// `pend`, and the next call first applies the rows that were accepted (npend), writes that state
// back once, then continues. The commit uses exactly the update the row already received, so the
// committed state is bit-identical to stepping the accepted rows one at a time.
#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

constexpr int kD = 128;
constexpr int kNT = 512;              // threads per block: 4 key groups x 128 value dims
constexpr int kJ = kD / 4;            // key rows per thread (32)

// pend buffer: header (256 B) | khat [R][VH][D] | delta [R][VH][D] | decay [R][VH] (fp32) |
// raw [R][NQKV] bf16 (pending conv inputs of the kernel-tier conv) | work [R][NQKV] bf16 (its
// convolved rows).
__host__ __device__ static inline size_t hdr_bytes() { return 256; }
__host__ __device__ static inline size_t area_floats(int vh) {
    return (size_t)kMaxRows * (2 * (size_t)vh * kD + vh);
}
size_t gdn_pend_raw_offset(int kh, int vh, int d) {
    (void)kh; (void)d;
    return (hdr_bytes() + area_floats(vh) * 4 + 255) & ~(size_t)255;
}
static size_t gdn_work_offset(int kh, int vh, int d) {
    return gdn_pend_raw_offset(kh, vh, d) + (size_t)kMaxRows * (2 * kh + vh) * d * 2;
}
size_t gdn_pend_bytes(int kh, int vh, int d) {
    const size_t nqkv = (size_t)(2 * kh + vh) * d;
    return gdn_work_offset(kh, vh, d) + (size_t)kMaxRows * nqkv * 2;
}
struct PendArea { float* khat; float* delta; float* decay; };
__device__ __forceinline__ PendArea pend_area(void* p, int vh) {
    float* b = (float*)((char*)p + hdr_bytes());
    PendArea v;
    v.khat = b;  b += (size_t)kMaxRows * vh * kD;
    v.delta = b; b += (size_t)kMaxRows * vh * kD;
    v.decay = b;
    return v;
}

__global__ __launch_bounds__(kNT) void k_gdn(GdnArgs a, int nr) {
    const int h = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int d = t & (kD - 1), g = t >> 7;
    const int ratio = a.vh / a.kh, kk = h / ratio;
    const int KD = a.kh * kD;
    const PendArea P = pend_area(a.pend, a.vh);     // pending rows: read first, then this call's rows
    const int npend = a.npend_ptr ? ld_uniform(a.npend_ptr) : a.npend_imm;

    __shared__ __attribute__((aligned(16))) float skp[kMaxRows][kD];
    __shared__ float sdp[kMaxRows][kD], sdc[kMaxRows];
    __shared__ float scv[kMaxRows][3 * kD];        // convolved q | k | v of this head (bf16 values)
    __shared__ float sz[kMaxRows][kD];
    __shared__ __attribute__((aligned(16))) float sq[kMaxRows][kD];
    __shared__ __attribute__((aligned(16))) float sk[kMaxRows][kD];
    __shared__ float pA[2][4][kD], pB[2][4][kD];
    __shared__ float smix[kMaxRows][kD];
    __shared__ float red[kMaxRows][2];
    __shared__ float srow[kMaxRows][4];          // per row: kq, beta, decay

    // ================= phase A: every global load of the block =================
    // (a) committed state slice
    const float* Sp = a.S + (size_t)h * kD * kD + (size_t)(g * kJ) * kD + d;
    float st[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) st[j] = Sp[(size_t)j * kD];
    // Every load below is unconditional (indices past the valid rows repeat a valid one, the values
    // are not used): a load under a condition is followed by its own wait, which serialises the
    // loads behind it into separate memory round trips.
    // (b) pending update vectors: thread t covers rows p = t/128 and p + 4
    float pk[2], pd[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int p = g + 4 * u;                    // < kMaxRows: inside the pend area
        pk[u] = P.khat[((size_t)p * a.vh + h) * kD + d];
        pd[u] = P.delta[((size_t)p * a.vh + h) * kD + d];
    }
    const float pdc = P.decay[(size_t)(t & (kMaxRows - 1)) * a.vh + h];
    // (c) channel t < 384 of this head: q (key head kk), k (kk), v (h); threads 384..511 the gate z
    const int cl = (t < 3 * kD) ? t : 0;
    const int ch = (cl < kD) ? kk * kD + cl : (cl < 2 * kD) ? KD + kk * kD + (cl - kD) : 2 * KD + h * kD + (cl - 2 * kD);
    const uint16_t* xsrc = (t < 3 * kD) ? a.qkv + ch : a.z + (size_t)h * kD + d;
    const size_t xstride = (t < 3 * kD) ? (size_t)a.qkv_stride : (size_t)a.z_stride;
    uint16_t xr[kMaxRows];
#pragma unroll
    for (int n = 0; n < kMaxRows; ++n) xr[n] = xsrc[(size_t)((n < nr) ? n : nr - 1) * xstride];
    // (d) the row scalars: prepared (decay, beta), or the a/b logits
    const int tr = (t < nr) ? t : nr - 1;
    float r_a, r_b;
    if (a.rowsc) {
        r_a = a.rowsc[(size_t)tr * a.vh + h];                              // decay
        r_b = a.rowsc[(size_t)(kMaxRows + tr) * a.vh + h];                 // beta
    } else {
        r_a = a.a[(size_t)tr * a.ab_stride + h];
        r_b = a.b[(size_t)tr * a.ab_stride + h];
    }
    const float Aexp = a.rowsc ? 0.0f : qexp(bf2f(a.A_log[h]));
    const float dtb = a.rowsc ? 0.0f : bf2f(a.dt_bias[h]);
    const float nw = bf2f(a.norm_w[(t & 63) + 64 * (wv & 1)]);

    // ================= phase B: on-chip work =================
    if (stopped(a.stop)) return;                // read once the loads are in flight
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int p = g + 4 * u;
        if (p < npend) { skp[p][d] = pk[u]; sdp[p][d] = pd[u]; }
    }
    if (t < npend) sdc[t] = pdc;
    if (t < nr) {
        if (a.rowsc) {
            srow[t][1] = r_b;
            srow[t][2] = r_a;
        } else {   // beta = sigmoid(b), decay = exp(-exp(A_log) softplus(a + dt))
            srow[t][1] = qsigmoid(r_b);
            srow[t][2] = qexp(-(Aexp * qsoftplus(r_a + dtb)));
        }
    }
    // every staged row is written (rows past nr hold copies of row nr - 1 and are not read): an
    // exit at nr would index the register array dynamically (a select chain per element)
#pragma unroll
    for (int n = 0; n < kMaxRows; ++n) {
        if (t < 3 * kD) scv[n][cl] = bf2f(xr[n]);
        else sz[n][d] = bf2f(xr[n]);
    }
    __syncthreads();

    // commit the accepted rows of the previous call, write the committed state back once
    for (int p = 0; p < npend; ++p) {
        const float dp = sdp[p][d], dc = sdc[p];
#pragma unroll
        for (int j4 = 0; j4 < kJ; j4 += 4) {
            const float4 kp = *(const float4*)&skp[p][g * kJ + j4];
            st[j4] = __builtin_fmaf(kp.x, dp, dc * st[j4]);
            st[j4 + 1] = __builtin_fmaf(kp.y, dp, dc * st[j4 + 1]);
            st[j4 + 2] = __builtin_fmaf(kp.z, dp, dc * st[j4 + 2]);
            st[j4 + 3] = __builtin_fmaf(kp.w, dp, dc * st[j4 + 3]);
        }
    }
    if (npend > 0) {
        float* Sw = a.S + (size_t)h * kD * kD + (size_t)(g * kJ) * kD + d;
#pragma unroll
        for (int j = 0; j < kJ; ++j) Sw[(size_t)j * kD] = st[j];
    }
    // q/k norms of whole rows, one wave per row: both 64-element halves, each reduced by the tree,
    // summed first half + second half; q^, k^ and k^.q^
    for (int n = wv; n < nr; n += kNT / 64) {
        const float q0 = scv[n][lane], q1 = scv[n][64 + lane];
        const float k0 = scv[n][kD + lane], k1 = scv[n][kD + 64 + lane];
        const float sq0 = tree64(q0 * q0), sq1 = tree64(q1 * q1);
        const float sk0 = tree64(k0 * k0), sk1 = tree64(k1 * k1);
        const float sx0 = tree64(q0 * k0), sx1 = tree64(q1 * k1);
        const float ssq = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq0 + sq1)));
        const float ssk = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sk0 + sk1)));
        const float invq = rsqrt_cr(ssq + 1e-6f) * 0.0883883476f;
        const float invk = rsqrt_cr(ssk + 1e-6f);
        const float kh0 = k0 * invk, kh1 = k1 * invk;
        sq[n][lane] = q0 * invq;
        sq[n][64 + lane] = q1 * invq;
        sk[n][lane] = kh0;
        sk[n][64 + lane] = kh1;
        P.khat[((size_t)n * a.vh + h) * kD + lane] = kh0;
        P.khat[((size_t)n * a.vh + h) * kD + 64 + lane] = kh1;
        if (lane == 0) srow[n][0] = ((sx0 + sx1) * invq) * invk;
    }
    __syncthreads();

    // the rows, in order: one barrier each (pA / pB alternate between two buffers)
    for (int n = 0; n < nr; ++n) {
        const float kq = srow[n][0], beta = srow[n][1], decay = srow[n][2];
        const float vv = scv[n][2 * kD + d];
        float accA = 0.0f, accB = 0.0f;
#pragma unroll
        for (int j4 = 0; j4 < kJ; j4 += 4) {
            const float4 k4 = *(const float4*)&sk[n][g * kJ + j4];
            const float4 q4 = *(const float4*)&sq[n][g * kJ + j4];
            accA = __builtin_fmaf(st[j4], k4.x, accA);
            accB = __builtin_fmaf(st[j4], q4.x, accB);
            accA = __builtin_fmaf(st[j4 + 1], k4.y, accA);
            accB = __builtin_fmaf(st[j4 + 1], q4.y, accB);
            accA = __builtin_fmaf(st[j4 + 2], k4.z, accA);
            accB = __builtin_fmaf(st[j4 + 2], q4.z, accB);
            accA = __builtin_fmaf(st[j4 + 3], k4.w, accA);
            accB = __builtin_fmaf(st[j4 + 3], q4.w, accB);
        }
        pA[n & 1][g][d] = accA;
        pB[n & 1][g][d] = accB;
        __syncthreads();
        const float A = ((pA[n & 1][0][d] + pA[n & 1][1][d]) + pA[n & 1][2][d]) + pA[n & 1][3][d];
        const float B = ((pB[n & 1][0][d] + pB[n & 1][1][d]) + pB[n & 1][2][d]) + pB[n & 1][3][d];
        const float delta = (vv - decay * A) * beta;
        const float mixed = __builtin_fmaf(delta, kq, decay * B);
        if (n + 1 < nr) {                           // the state after the last row is never needed
#pragma unroll
            for (int j4 = 0; j4 < kJ; j4 += 4) {
                const float4 k4 = *(const float4*)&sk[n][g * kJ + j4];
                st[j4] = __builtin_fmaf(k4.x, delta, decay * st[j4]);
                st[j4 + 1] = __builtin_fmaf(k4.y, delta, decay * st[j4 + 1]);
                st[j4 + 2] = __builtin_fmaf(k4.z, delta, decay * st[j4 + 2]);
                st[j4 + 3] = __builtin_fmaf(k4.w, delta, decay * st[j4 + 3]);
            }
        }
        if (g == 0) {
            P.delta[((size_t)n * a.vh + h) * kD + d] = delta;
            smix[n][d] = mixed;
        }
        if (t == 0) P.decay[(size_t)n * a.vh + h] = decay;
    }
    __syncthreads();

    // output norm + gate + quantize, row n on the wave pair (2m, 2m+1), element e = 64 (w&1) + lane
    const int e = 64 * (wv & 1) + lane;
    for (int n = wv >> 1; n < nr; n += 4) {
        const float mx = smix[n][e];
        const float r3 = tree64(mx * mx);
        if (lane == 0) red[n][wv & 1] = r3;
    }
    __syncthreads();
    for (int n = wv >> 1; n < nr; n += 4) {
        const float mx = smix[n][e];
        const float inv = rsqrt_cr((red[n][0] + red[n][1]) * (1.0f / (float)kD) + a.eps);
        const float y = mx * inv * nw * qsilu(sz[n][e]);
        const uint16_t yb = f2bf(y);
        const size_t k = (size_t)n * a.out_stride + (size_t)h * kD + e;
        a.out[k] = yb;
        if (a.xq) {   // the per-16 quantizer with g = 1/in_scale (s = mx g / 127, 1/s -> g / s)
            const float g = (a.in_scale > 0.0f) ? 1.0f / a.in_scale : 1.0f;
            const float yv = bf2f(yb);
            const float m16 = max_xor(fabsf(yv), 16);
            const float sc = m16 * g * (1.0f / 127.0f);
            const float qi = (sc > 0.0f) ? (g / sc) : 0.0f;
            a.xq[k] = qcode(yv, qi);
            if ((e & 15) == 0) a.xs[k >> 4] = sc;
        }
    }
}

// Prefill scan: the same per-row arithmetic as k_gdn over all nrows rows of a chunk, with the
// value columns spread over waves instead of the key rows over a block. Value columns of the
// delta rule are independent given the row's (k^, q^, beta, decay), so a wave owns 16 of them:
// lane 16 g + c holds key rows 32g..32g+31 of column c, and the four key groups' partial sums
// S^T k, S^T q meet by lane swaps in the order ((p0 + p1) + p2) + p3, which is k_gdn's order. No
// barrier per row: a block (WPB waves, 16 WPB columns of one head) only synchronises per batch
// of staged rows, to share the q/k norms. The state stays in registers from the first row to the
// last and is written back once. Each row's mixed values go to `mix` [nrows][vh*128] fp32;
// k_gdn_gnorm applies the gated RMSNorm afterwards (it needs the head's 128 columns, which live in
// several blocks). Row scalars: decay at rowsc[n vh + h], beta at rowsc[(nrows + n) vh + h].
// q/k norms of the scan's rows, outside the scan (they do not depend on the state): one wave per
// (row, key head), k_gdn's arithmetic (two 64-lane trees per sum, first half + second half).
// qk [nrows][kh][256]: q^ (128) then k^ (128); kq [nrows][kh]: k^.q^.
__global__ __launch_bounds__(256) void k_gdn_qknorm(const uint16_t* __restrict__ qkv, int qkv_stride, int kh,
                                                    int nrows, float* __restrict__ qk, float* __restrict__ kq) {
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);     // (row, key head) pair
    if (u >= nrows * kh) return;
    const int row = u / kh, kk = u - row * kh;
    const uint16_t* src = qkv + (size_t)row * qkv_stride;
    const int KD = kh * kD;
    const float q0 = bf2f(src[kk * kD + lane]), q1 = bf2f(src[kk * kD + 64 + lane]);
    const float k0 = bf2f(src[KD + kk * kD + lane]), k1 = bf2f(src[KD + kk * kD + 64 + lane]);
    const float sq0 = tree64(q0 * q0), sq1 = tree64(q1 * q1);
    const float sk0 = tree64(k0 * k0), sk1 = tree64(k1 * k1);
    const float sx0 = tree64(q0 * k0), sx1 = tree64(q1 * k1);
    const float ssq = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq0 + sq1)));
    const float ssk = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sk0 + sk1)));
    const float invq = rsqrt_cr(ssq + 1e-6f) * 0.0883883476f;
    const float invk = rsqrt_cr(ssk + 1e-6f);
    float* d = qk + (size_t)u * 2 * kD;
    d[lane] = q0 * invq;
    d[64 + lane] = q1 * invq;
    d[kD + lane] = k0 * invk;
    d[kD + 64 + lane] = k1 * invk;
    if (lane == 0) kq[u] = ((sx0 + sx1) * invq) * invk;
}
#ifndef Q27X_SCAN_WPB
#define Q27X_SCAN_WPB 4
#endif
constexpr int kScanWPB = Q27X_SCAN_WPB;  // waves per block
// ((p0 + p1) + p2) + p3 over the lanes c, 16 + c, 32 + c, 48 + c (p_g in lane 16 g + c), exact in
// the lanes of group 0 (the other lanes hold partial values). The gfx950 lane swaps exchange
// 16-lane rows 0<->1, 2<->3 and the 32-lane halves; the second result holds the partner's value
// in the even rows / lower half.
__device__ __forceinline__ float key_group_sum_g0(float x) {
    const float a = __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
    const float b = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false)[1]);
    const float c = __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(b), __float_as_uint(b), false, false)[1]);
    return ((x + a) + b) + c;      // group 0: a = p1, b = p2, c = p3 (row 1's b is row 3's x)
}
// group 0's value in every lane of its column: row 0 -> row 1 by a 16-lane swap, rows 0, 1 -> rows
// 2, 3 by a 32-lane swap (the first result holds the partner's value in the odd rows / upper half)
__device__ __forceinline__ float from_group0(float s) {
    const int g = (threadIdx.x >> 4) & 3;
    const float t = __uint_as_float(__builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false, false)[0]);
    const float u = (g == 1) ? t : s;
    const float w = __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(u), __float_as_uint(u), false, false)[0]);
    return (g >= 2) ? w : u;
}
template <int WPB>
__global__ __launch_bounds__(64 * WPB) void k_gdn_scan(GdnArgs a, const float* __restrict__ qk,
                                                      const float* __restrict__ kqv, float* __restrict__ mix,
                                                      int nrows) {
    constexpr int NT = 64 * WPB, NC = 16 * WPB;          // threads, value columns of the block
    constexpr int R = 8 * WPB;                           // rows staged per batch
    constexpr int CPT = 2 * kD / NT;                     // q|k channels loaded per thread
    constexpr int BPH = kD / NC;                         // blocks per head
    static_assert(CPT >= 1 && CPT * NT == 2 * kD && BPH * NC == kD, "1, 2 or 4 waves per block");
    const int h = blockIdx.x / BPH, part = blockIdx.x % BPH;
    const int t = threadIdx.x, lane = t & 63, wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int g = lane >> 4, cw = 16 * wv + (lane & 15);      // column within the block's NC
    const int col = NC * part + cw;
    const int ratio = a.vh / a.kh, kk = h / ratio;
    const int KD = a.kh * kD;
    const size_t mstride = (size_t)a.vh * kD;
    __shared__ float sv[R][NC];                  // v of the block's columns
    __shared__ __attribute__((aligned(16))) float sq[R][kD];
    __shared__ __attribute__((aligned(16))) float sk[R][kD];
    __shared__ float srow[R][4];                 // per row: kq, beta, decay
    __shared__ float smix[R][NC];
    float* Sp = a.S + (size_t)h * kD * kD + (size_t)(g * kJ) * kD + col;
    float st[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) st[j] = Sp[(size_t)j * kD];
    // thread t loads the normed q^|k^ values t + NT i of the key head (< 128: q^, else k^) and v
    // column NC part + t % NC
    const size_t chv = (size_t)2 * KD + (size_t)h * kD + NC * part + (t % NC);
    float xr[R][CPT];
    uint16_t xv[R];
    float r_a = 0.0f, r_b = 0.0f, r_kq = 0.0f;
    // unconditional loads (rows past the last repeat it; every thread loads a v column): a load
    // under a condition is followed by its own wait, which would serialise the batch's loads
    auto load = [&](int r0) {
#pragma unroll
        for (int n = 0; n < R; ++n) {
            const int rn = (r0 + n < nrows) ? r0 + n : nrows - 1;
#pragma unroll
            for (int i = 0; i < CPT; ++i) xr[n][i] = qk[((size_t)rn * a.kh + kk) * 2 * kD + t + NT * i];
            xv[n] = a.qkv[(size_t)rn * a.qkv_stride + chv];
        }
        const int rt = (r0 + (t % R) < nrows) ? r0 + (t % R) : nrows - 1;
        r_a = a.rowsc[(size_t)rt * a.vh + h];
        r_b = a.rowsc[(size_t)(nrows + rt) * a.vh + h];
        r_kq = kqv[(size_t)rt * a.kh + kk];
    };
    load(0);
    for (int r0 = 0; r0 < nrows; r0 += R) {
        const int nr = (nrows - r0 < R) ? nrows - r0 : R;
        __syncthreads();                            // the previous batch is written out
        if (t < nr) { srow[t][0] = r_kq; srow[t][1] = r_b; srow[t][2] = r_a; }
        // every staged row is written (rows past nr hold copies of the last row and are not read):
        // an exit at nr would index the register arrays dynamically (a select chain per element)
#pragma unroll
        for (int n = 0; n < R; ++n) {
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                const int c = t + NT * i;
                if (c < kD) sq[n][c] = xr[n][i];
                else sk[n][c - kD] = xr[n][i];
            }
            if (t < NC) sv[n][t] = bf2f(xv[n]);
        }
        if (r0 + R < nrows) load(r0 + R);            // next batch in flight during this one
        __syncthreads();
        // rows in pairs: everything a row reads from LDS is requested while the row before it
        // computes (a row's own reads would make every wait cover the prefetch behind them)
        struct RowIn { float k[kJ], q[kJ]; float kq, beta, decay, v; };
        auto lds_row = [&](int n, RowIn& r) {
#pragma unroll
            for (int j4 = 0; j4 < kJ; j4 += 4) {
                const float4 k4 = *(const float4*)&sk[n][g * kJ + j4];
                const float4 q4 = *(const float4*)&sq[n][g * kJ + j4];
                r.k[j4] = k4.x; r.k[j4 + 1] = k4.y; r.k[j4 + 2] = k4.z; r.k[j4 + 3] = k4.w;
                r.q[j4] = q4.x; r.q[j4 + 1] = q4.y; r.q[j4 + 2] = q4.z; r.q[j4 + 3] = q4.w;
            }
            r.kq = srow[n][0]; r.beta = srow[n][1]; r.decay = srow[n][2];
            r.v = sv[n][cw];
        };
        auto do_row = [&](int n, const RowIn& r) {
            float accA = 0.0f, accB = 0.0f;
#pragma unroll
            for (int j = 0; j < kJ; ++j) {
                accA = __builtin_fmaf(st[j], r.k[j], accA);
                accB = __builtin_fmaf(st[j], r.q[j], accB);
            }
            const float A = from_group0(key_group_sum_g0(accA));
            const float delta = (r.v - r.decay * A) * r.beta;
#pragma unroll
            for (int j = 0; j < kJ; ++j) st[j] = __builtin_fmaf(r.k[j], delta, r.decay * st[j]);
            const float B = key_group_sum_g0(accB);                 // needed in group 0 only
            const float mixed = __builtin_fmaf(delta, r.kq, r.decay * B);
            if (g == 0) smix[n][cw] = mixed;
        };
        // (the prefetches are unconditional, of row min(n, nr - 1), so that every path through the
        // loop has the same reads in flight and the waits count only the reads a row needs)
        RowIn ra, rb;
        lds_row(0, ra);
        for (int n = 0; n < nr; n += 2) {
            lds_row((n + 1 < nr) ? n + 1 : nr - 1, rb);
            do_row(n, ra);
            lds_row((n + 2 < nr) ? n + 2 : nr - 1, ra);
            if (n + 1 < nr) do_row(n + 1, rb);
        }
        __syncthreads();
        for (int i = t; i < nr * NC; i += NT) {
            const int n = i / NC, c = i % NC;
            mix[(size_t)(r0 + n) * mstride + (size_t)h * kD + NC * part + c] = smix[n][c];
        }
    }
#pragma unroll
    for (int j = 0; j < kJ; ++j) Sp[(size_t)j * kD] = st[j];
}
// gated RMSNorm of the scan's rows (k_gdn's arithmetic: two 64-lane trees of mixed^2, their sum
// over 128, rsqrt; y = mixed inv norm_w SiLU(z) -> bf16). One 128-thread block per (head, row).
__global__ __launch_bounds__(kD) void k_gdn_gnorm(const float* __restrict__ mix, const uint16_t* __restrict__ z,
                                                  int z_stride, const uint16_t* __restrict__ norm_w, float eps,
                                                  int vh, uint16_t* __restrict__ out, int out_stride) {
    const int h = blockIdx.x, row = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    __shared__ float red[2];
    const float mx = mix[(size_t)row * vh * kD + (size_t)h * kD + t];
    const float zz = bf2f(z[(size_t)row * z_stride + (size_t)h * kD + t]);
    const float nw = bf2f(norm_w[t]);
    const float r3 = tree64(mx * mx);
    if (lane == 0) red[w] = r3;
    __syncthreads();
    const float inv = rsqrt_cr((red[0] + red[1]) * (1.0f / (float)kD) + eps);
    out[(size_t)row * out_stride + (size_t)h * kD + t] = f2bf(mx * inv * nw * qsilu(zz));
}
int launch_gdn_scan(const GdnArgs& a, int nrows, float* qk, float* kq, float* mix, hipStream_t s) {
    if (a.d != kD || a.kh < 1 || a.vh % a.kh || nrows < 1 || !a.qkv || !a.z || !a.S || !a.rowsc || !a.out ||
        !a.norm_w || !mix || !qk || !kq || nrows > 65535) {
        set_error("gdn scan: unsupported shape or null argument (d=%d kh=%d vh=%d rows=%d)", a.d, a.kh, a.vh, nrows);
        return Q27X_E_SHAPE;
    }
    hipLaunchKernelGGL(k_gdn_qknorm, dim3((unsigned)((nrows * a.kh + 3) / 4)), dim3(256), 0, s, a.qkv, a.qkv_stride,
                       a.kh, nrows, qk, kq);
    Q27X_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_gdn_scan<kScanWPB>, dim3(a.vh * (kD / (16 * kScanWPB))), dim3(64 * kScanWPB), 0, s, a,
                       (const float*)qk, (const float*)kq, mix, nrows);
    Q27X_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_gdn_gnorm, dim3(a.vh, nrows), dim3(kD), 0, s, (const float*)mix, a.z, a.z_stride, a.norm_w,
                       a.eps, a.vh, a.out, a.out_stride);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

int launch_gdn(const GdnArgs& a, int nr, hipStream_t s) {
    if (a.d != kD || a.kh < 1 || a.vh % a.kh || nr < 1 || nr > kMaxRows || !a.qkv || !a.z || !a.S || !a.pend ||
        !a.out || !a.norm_w) {
        set_error("gdn: unsupported shape or null argument (d=%d kh=%d vh=%d nr=%d)", a.d, a.kh, a.vh, nr);
        return Q27X_E_SHAPE;
    }
    if (a.xq && a.out_stride % 16) { set_error("gdn: out_stride must be a multiple of 16"); return Q27X_E_ARG; }
    if (!a.rowsc && (!a.a || !a.b || !a.A_log || !a.dt_bias)) {
        set_error("gdn: the row scalars or the a/b logits with A_log and dt_bias are required");
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_gdn, dim3(a.vh), dim3(kNT), 0, s, a, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
int gdn_set_lds_limit() { return Q27X_OK; }

// conv + SiLU with the deferred shift-register commit as a standalone kernel (the kernel-tier
// entry; the engine convolves inside k_gdn)
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
    if (nr == 0) return;   // commit only
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

// Commit only: apply the npend pending rows of `pend` to S (the update each row already received,
// the same fmaf as k_gdn's commit), write S back, and leave nothing pending. One block per value
// head, thread (g, d) holds key rows 32 g .. 32 g + 31 of value column d.
constexpr int kCommitT = kNT;        // commit kernel: thread (g, d), key group g < 4, column d < 128
__global__ __launch_bounds__(kCommitT) void k_gdn_commit(float* __restrict__ S, const void* pend, int vh, int npend) {
    const int h = blockIdx.x, t = threadIdx.x, d = t & (kD - 1), g = t >> 7;
    const PendArea P = pend_area(const_cast<void*>(pend), vh);
    float* Sp = S + (size_t)h * kD * kD + (size_t)(g * kJ) * kD + d;
    float st[kJ];
#pragma unroll
    for (int j = 0; j < kJ; ++j) st[j] = Sp[(size_t)j * kD];
    for (int p = 0; p < npend; ++p) {
        const float dp = P.delta[((size_t)p * vh + h) * kD + d], dc = P.decay[(size_t)p * vh + h];
        const float* kp = P.khat + ((size_t)p * vh + h) * kD + g * kJ;
#pragma unroll
        for (int j = 0; j < kJ; ++j) st[j] = __builtin_fmaf(kp[j], dp, dc * st[j]);
    }
#pragma unroll
    for (int j = 0; j < kJ; ++j) Sp[(size_t)j * kD] = st[j];
}

}  // namespace q27x

using namespace q27x;
extern "C" size_t q27x_gdn_pend_bytes(int kh, int vh, int d, int max_rows) {
    (void)max_rows;
    return gdn_pend_bytes(kh, vh, d);
}

// Kernel-tier entry: conv (deferred commit, in place on conv_hist) then the recurrence. The
// conv'd rows go to the work area at the end of `pend`, so the call allocates nothing.
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
    uint16_t* conv_buf = (uint16_t*)((char*)pend + gdn_work_offset(kh, vh, d));
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

// Kernel-tier commit without new rows: the conv shift registers and S take the npend pending rows
// that q27x_gdn_verify left in `pend` (the accepted prefix of its last call). Afterwards nothing is
// pending: the next q27x_gdn_verify call passes npend = 0.
extern "C" int q27x_gdn_commit(float* S, uint16_t* conv_hist, void* pend, int npend, int kh, int vh, int d,
                               q27x_stream_t s) {
    if (!S || !conv_hist || !pend || npend < 0 || npend > kMaxRows || d != 128 || kh < 1 || vh % kh) {
        set_error("q27x_gdn_commit: bad arguments");
        return Q27X_E_ARG;
    }
    if (npend == 0) return Q27X_OK;
    const int nconv = (2 * kh + vh) * d;
    uint16_t* pend_raw = (uint16_t*)((char*)pend + gdn_pend_raw_offset(kh, vh, d));
    int rc = launch_gdn_conv(nullptr, 0, nullptr, 0, nconv, nullptr, conv_hist, pend_raw, nullptr, npend, 0,
                             (hipStream_t)s);
    if (rc) return rc;
    hipLaunchKernelGGL(k_gdn_commit, dim3(vh), dim3(kCommitT), 0, (hipStream_t)s, S, (const void*)pend, vh, npend);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}
