// k_proj.hip -- W8A8 projection of NR <= 8 rows and the bf16 GEMV (lm_head, GDN a/b).
//
// Memory-bound: one pass over the weights serves every verify row. A wave owns RPW weight rows
// at a time; lane l streams 16 B of each row per 1024-element step (the 64 lanes of a step read
// one contiguous 1 KiB run per row, non-temporal), so slab s = 64*step + lane of the row meets
// the same slab of every activation row staged once per block in LDS. Per slab:
//   int d = sdot4 x 4 (exact int32), acc = fmaf((float)d, ws64 * xs16, acc)
// then the 64 lane sums meet in the shfl_down tree -- the reference's order
// (src/q27_fp8.hip:3814-3871), kept so results match its host restatement bit for bit.
// The grid is persistent-ish (grid-stride over row tiles) with the next tile's weights
// prefetched into registers while the current tile is reduced and stored.
#include "q27x_dev.h"
#include "q27x_int.h"

namespace q27x {

template <int NR, int NSTEP, int RPW, int NW, int EPI>
__global__ __launch_bounds__(NW * 64) void k_proj(ProjArgs a) {
    constexpr int NT = NW * 64;
    constexpr int TILE = NW * RPW;
    constexpr int SL = NSTEP * 64;                  // slabs per staged activation row
    __shared__ uint4 sx[NR * SL];
    __shared__ float ssc[NR * SL];
    __shared__ float tout[NR][TILE];
    if (a.stop && *a.stop) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = a.K, nslab = K >> 4, ng64 = K >> 6;
    for (int i = threadIdx.x; i < NR * SL; i += NT) {
        const int n = i / SL, s = i - n * SL;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        float sc = 0.0f;
        if (s < nslab) {
            v = *(const uint4*)(a.xq + (size_t)n * a.xst + 16 * s);
            sc = a.xs[(size_t)n * (a.xst >> 4) + s];
        }
        sx[i] = v;
        ssc[i] = sc;
    }
    __syncthreads();
    const int ntiles = (a.rows + TILE - 1) / TILE;
    uint4 wv[RPW][NSTEP];
    float wsv[RPW][NSTEP];
    auto load = [&](int tl, uint4 (&W_)[RPW][NSTEP], float (&S_)[RPW][NSTEP]) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            int row = tl * TILE + wave * RPW + r;
            row = row < a.rows ? row : a.rows - 1;
            const int8_t* wp = a.W + (size_t)row * K;
            const float* sp = a.WS + (size_t)row * ng64;
#pragma unroll
            for (int t = 0; t < NSTEP; ++t) {
                const int s = t * 64 + lane;
                if (s < nslab) { W_[r][t] = ld_nt16(wp + 16 * s); S_[r][t] = sp[s >> 2]; }
                else { W_[r][t] = make_uint4(0u, 0u, 0u, 0u); S_[r][t] = 0.0f; }
            }
        }
    };
    int tile = blockIdx.x;
    if (tile < ntiles) load(tile, wv, wsv);
    for (; tile < ntiles; tile += gridDim.x) {
        uint4 wn[RPW][NSTEP];
        float wsn[RPW][NSTEP];
        const int next = tile + gridDim.x;
        if (next < ntiles) load(next, wn, wsn);
        float acc[RPW][NR];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = 0.0f;
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
            const int s = t * 64 + lane;
            if (s < nslab) {
#pragma unroll
                for (int n = 0; n < NR; ++n) {
                    const uint4 xa = sx[n * SL + s];
                    const float sa = ssc[n * SL + s];
#pragma unroll
                    for (int r = 0; r < RPW; ++r) {
                        const int d = dot16(wv[r][t], xa);
                        acc[r][n] = __builtin_fmaf((float)d, wsv[r][t] * sa, acc[r][n]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = tree64(acc[r][n]);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int n = 0; n < NR; ++n) tout[n][wave * RPW + r] = acc[r][n] * a.alpha;
        }
        __syncthreads();
        const int row0 = tile * TILE;
        if (EPI == EPI_STORE) {
            for (int i = threadIdx.x; i < NR * TILE; i += NT) {
                const int n = i / TILE, j = i - n * TILE, row = row0 + j;
                if (row >= a.rows) continue;
                float v = tout[n][j];
                if (a.res) {
                    const float rv = a.res_bf16 ? bf2f(((const uint16_t*)a.res)[(size_t)n * a.rstride + row])
                                                : ((const float*)a.res)[(size_t)n * a.rstride + row];
                    if (a.res_round) v = bfr(v);
                    v = v + a.rs * rv;
                }
                if (a.out_bf16) ((uint16_t*)a.y)[(size_t)n * a.ystride + row] = f2bf(v);
                else ((float*)a.y)[(size_t)n * a.ystride + row] = v;
            }
        } else if (EPI == EPI_GDN_IN) {
            const int j = threadIdx.x;
            const int row = row0 + j;
            if (j < TILE && row < a.rows) {
                if (row < a.nconv) {
                    // k_gdn_conv_tp_tile (src/q27_gdn.hip:411-439): raw bf16 shift register,
                    // first tap a plain product, fmaf for taps 1..3, SiLU, bf16. The pending rows
                    // of the previous call are shifted in first (deferred commit).
                    const int c = row;
                    const int npend = a.npend_ptr ? *a.npend_ptr : a.npend_imm;
                    uint16_t h0 = a.conv_hist[3 * c], h1 = a.conv_hist[3 * c + 1], h2 = a.conv_hist[3 * c + 2];
                    for (int p = 0; p < npend; ++p) {
                        h0 = h1; h1 = h2; h2 = a.pend_raw[(size_t)p * a.nconv + c];
                    }
                    a.conv_hist[3 * c] = h0; a.conv_hist[3 * c + 1] = h1; a.conv_hist[3 * c + 2] = h2;
                    const float w0 = bf2f(a.conv_w[4 * c]), w1 = bf2f(a.conv_w[4 * c + 1]);
                    const float w2 = bf2f(a.conv_w[4 * c + 2]), w3 = bf2f(a.conv_w[4 * c + 3]);
#pragma unroll
                    for (int n = 0; n < NR; ++n) {
                        const uint16_t x = f2bf(tout[n][j]);
                        float acc = bf2f(h0) * w0;
                        acc = __builtin_fmaf(bf2f(h1), w1, acc);
                        acc = __builtin_fmaf(bf2f(h2), w2, acc);
                        acc = __builtin_fmaf(bf2f(x), w3, acc);
                        h0 = h1; h1 = h2; h2 = x;
                        a.pend_raw[(size_t)n * a.nconv + c] = x;
                        a.conv_out[(size_t)n * a.conv_stride + c] = f2bf(qsilu(acc));
                    }
                } else {
#pragma unroll
                    for (int n = 0; n < NR; ++n)
                        a.z_out[(size_t)n * a.z_stride + (row - a.nconv)] = f2bf(tout[n][j]);
                }
            }
        } else {   // EPI_SWIGLU: tile = [16 gate rows | 16 up rows] -> 16 outputs, one group
            const int i = threadIdx.x;
            if (i < NR * 16) {
                const int n = i >> 4, j = i & 15;
                const float g = tout[n][j], u = tout[n][16 + j];
                const float sw = g / (1.0f + qexp(-g));
                const float v = sw * u * a.gscale;
                const float mx = max_xor(fabsf(v), 16);
                const float sc = mx * (1.0f / 127.0f);
                const float inv = (sc > 0.0f) ? (1.0f / sc) : 0.0f;
                a.act_q[(size_t)n * a.act_stride + tile * 16 + j] = qcode(v, inv);
                if (j == 0) a.act_s[(size_t)n * (a.act_stride >> 4) + tile] = sc;
            }
        }
        __syncthreads();
        if (next < ntiles) {
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int t = 0; t < NSTEP; ++t) { wv[r][t] = wn[r][t]; wsv[r][t] = wsn[r][t]; }
        }
    }
}

static int g_ncu = 0;
static int num_cus() {
    if (!g_ncu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 256;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return 256;
        g_ncu = p.multiProcessorCount > 0 ? p.multiProcessorCount : 256;
    }
    return g_ncu;
}

template <int NR, int NSTEP, int RPW, int NW, int EPI>
static int run_proj(const ProjArgs& a, hipStream_t s, int blocks_per_cu) {
    constexpr int TILE = NW * RPW;
    const int ntiles = (a.rows + TILE - 1) / TILE;
    int grid = num_cus() * blocks_per_cu;
    if (grid > ntiles) grid = ntiles;
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL((k_proj<NR, NSTEP, RPW, NW, EPI>), dim3(grid), dim3(NW * 64), 0, s, a);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

// Shape router. NSTEP = ceil(K/1024). The LDS stage is NR*NSTEP*1280 B; K = 17408 at NR = 8
// (174 KB) is split by the caller into two launches of 4 rows.
template <int NR, int EPI>
static int route_k(const ProjArgs& a, hipStream_t s) {
    const int ns = (a.K + 1023) / 1024;
    if constexpr (EPI == EPI_SWIGLU) {
        if (ns == 1) return run_proj<NR, 1, 4, 8, EPI>(a, s, 2);
        if (ns == 2) return run_proj<NR, 2, 4, 8, EPI>(a, s, 2);
        if (ns == 5) return run_proj<NR, 5, 4, 8, EPI>(a, s, 2);
        return -2;
    }
    else if constexpr (EPI == EPI_GDN_IN) {
        if (ns == 1) return run_proj<NR, 1, 2, 4, EPI>(a, s, 4);
        if (ns == 2) return run_proj<NR, 2, 2, 4, EPI>(a, s, 4);
        if (ns == 5) return run_proj<NR, 5, 2, 4, EPI>(a, s, 4);
        return -2;
    } else {
    switch (ns) {
        case 1: return run_proj<NR, 1, 2, 4, EPI>(a, s, 4);
        case 2: return run_proj<NR, 2, 2, 4, EPI>(a, s, 4);
        case 4: return run_proj<NR, 4, 2, 4, EPI>(a, s, 4);
        case 5: return run_proj<NR, 5, 2, 4, EPI>(a, s, 4);
        case 6: return run_proj<NR, 6, 2, 4, EPI>(a, s, 4);
        case 17:
            if constexpr (NR <= 4) return run_proj<NR, 17, 1, 4, EPI>(a, s, 2);
            return -2;
        default: return -2;
    }
    }
}

template <int EPI>
static int route_nr(const ProjArgs& a, int nr, hipStream_t s) {
    switch (nr) {
        case 1: return route_k<1, EPI>(a, s);
        case 2: return route_k<2, EPI>(a, s);
        case 3: return route_k<3, EPI>(a, s);
        case 4: return route_k<4, EPI>(a, s);
        case 5: return route_k<5, EPI>(a, s);
        case 6: return route_k<6, EPI>(a, s);
        case 7: return route_k<7, EPI>(a, s);
        case 8: return route_k<8, EPI>(a, s);
        default: return -2;
    }
}

int launch_proj(const ProjArgs& a, int epi, int nr, hipStream_t s) {
    if (!a.W || !a.WS || !a.xq || !a.xs || a.rows < 1 || a.K < 64 || (a.K & 63) || nr < 1 || nr > kMaxRows) {
        set_error("proj: bad arguments (rows=%d K=%d nr=%d)", a.rows, a.K, nr);
        return Q27X_E_ARG;
    }
    if ((a.xst & 15) || a.xst < a.K) { set_error("proj: activation stride %d must be >= K and a multiple of 16", a.xst); return Q27X_E_ARG; }
    int rc;
    if (epi == EPI_STORE && a.K > 8192 && nr > 4) {   // LDS stage limit: two launches of <= 4 rows
        ProjArgs b = a;
        rc = route_nr<EPI_STORE>(b, 4, s);
        if (rc) return rc;
        b.xq = a.xq + (size_t)4 * a.xst;
        b.xs = a.xs + (size_t)4 * (a.xst >> 4);
        const size_t esz = a.out_bf16 ? 2 : 4;
        b.y = (char*)a.y + (size_t)4 * a.ystride * esz;
        if (a.res) b.res = (const char*)a.res + (size_t)4 * a.rstride * (a.res_bf16 ? 2 : 4);
        rc = route_nr<EPI_STORE>(b, nr - 4, s);
    } else if (epi == EPI_STORE) rc = route_nr<EPI_STORE>(a, nr, s);
    else if (epi == EPI_GDN_IN) rc = route_nr<EPI_GDN_IN>(a, nr, s);
    else rc = route_nr<EPI_SWIGLU>(a, nr, s);
    if (rc == -2) { set_error("proj: no kernel for K=%d nr=%d epi=%d", a.K, nr, epi); return Q27X_E_SHAPE; }
    return rc;
}

// ---------------------------------------------------------------- int32 slab partials
__global__ __launch_bounds__(256) void k_proj_partials(const int8_t* __restrict__ W, int rows, int K,
                                                       const int8_t* __restrict__ xq, int xst,
                                                       int32_t* __restrict__ part, int nr) {
    const int nslab = K >> 4;
    const long long total = (long long)nr * rows * nslab;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long long)gridDim.x * 256) {
        const int s = (int)(i % nslab);
        const long long rn = i / nslab;
        const int r = (int)(rn % rows), n = (int)(rn / rows);
        const uint4 w = *(const uint4*)(W + (size_t)r * K + 16 * s);
        const uint4 x = *(const uint4*)(xq + (size_t)n * xst + 16 * s);
        part[i] = dot16(w, x);
    }
}

// ---------------------------------------------------------------- bf16 GEMV
// Chunk c of 8 bf16 (16 B) belongs to lane c%64 at step c/64; fmaf per element in order; shfl
// tree. Activations staged as fp32 in LDS. MODE 1 keeps a running (value, index) argmax per row
// (non-finite filtered, ties to the lowest index: src/q27_elem.hip:226-236) and writes one
// partial per block.
__device__ __forceinline__ void am_merge(float& bv, uint32_t& bi, float v, uint32_t i) {
    const bool take = (v > bv) || (v == bv && i < bi);
    bv = take ? v : bv;
    bi = take ? i : bi;
}
__device__ __forceinline__ bool finitef(float v) { return (__float_as_uint(v) & 0x7F800000u) != 0x7F800000u; }

template <int NR, int NSTEP, int RPW, int MODE>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs a) {
    constexpr int NW = 4, NT = 256, TILE = NW * RPW, CH = NSTEP * 64;
    __shared__ float sxf[NR * CH * 8];
    __shared__ float tout[NR][TILE];
    __shared__ float bvs[NR][NW];
    __shared__ uint32_t bis[NR][NW];
    if (a.stop && *a.stop) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int K = a.K, nch = K >> 3;
    for (int i = threadIdx.x; i < NR * CH * 8; i += NT) {
        const int n = i / (CH * 8), k = i - n * (CH * 8);
        sxf[i] = (k < K) ? bf2f(a.x[(size_t)n * a.xst + k]) : 0.0f;
    }
    __syncthreads();
    float bv[NR];
    uint32_t bi[NR];
#pragma unroll
    for (int n = 0; n < NR; ++n) { bv[n] = -__builtin_huge_valf(); bi[n] = 0xFFFFFFFFu; }
    const int ntiles = (a.rows + TILE - 1) / TILE;
    uint4 wv[RPW][NSTEP];
    auto load = [&](int tl, uint4 (&W_)[RPW][NSTEP]) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            int row = tl * TILE + wave * RPW + r;
            row = row < a.rows ? row : a.rows - 1;
            const uint16_t* wp = a.W + (size_t)row * K;
#pragma unroll
            for (int t = 0; t < NSTEP; ++t) {
                const int c = t * 64 + lane;
                W_[r][t] = (c < nch) ? ld_nt16(wp + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
            }
        }
    };
    int tile = blockIdx.x;
    if (tile < ntiles) load(tile, wv);
    for (; tile < ntiles; tile += gridDim.x) {
        uint4 wn[RPW][NSTEP];
        const int next = tile + gridDim.x;
        if (next < ntiles) load(next, wn);
        float acc[RPW][NR];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = 0.0f;
#pragma unroll
        for (int t = 0; t < NSTEP; ++t) {
            const int c = t * 64 + lane;
            if (c < nch) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const uint4 w = wv[r][t];
                    float wf[8];
                    wf[0] = __uint_as_float(w.x << 16); wf[1] = __uint_as_float(w.x & 0xFFFF0000u);
                    wf[2] = __uint_as_float(w.y << 16); wf[3] = __uint_as_float(w.y & 0xFFFF0000u);
                    wf[4] = __uint_as_float(w.z << 16); wf[5] = __uint_as_float(w.z & 0xFFFF0000u);
                    wf[6] = __uint_as_float(w.w << 16); wf[7] = __uint_as_float(w.w & 0xFFFF0000u);
#pragma unroll
                    for (int n = 0; n < NR; ++n) {
                        const float4 x0 = *(const float4*)&sxf[n * CH * 8 + 8 * c];
                        const float4 x1 = *(const float4*)&sxf[n * CH * 8 + 8 * c + 4];
                        float v = acc[r][n];
                        v = __builtin_fmaf(wf[0], x0.x, v); v = __builtin_fmaf(wf[1], x0.y, v);
                        v = __builtin_fmaf(wf[2], x0.z, v); v = __builtin_fmaf(wf[3], x0.w, v);
                        v = __builtin_fmaf(wf[4], x1.x, v); v = __builtin_fmaf(wf[5], x1.y, v);
                        v = __builtin_fmaf(wf[6], x1.z, v); v = __builtin_fmaf(wf[7], x1.w, v);
                        acc[r][n] = v;
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int n = 0; n < NR; ++n) acc[r][n] = tree64(acc[r][n]);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int n = 0; n < NR; ++n) tout[n][wave * RPW + r] = acc[r][n];
        }
        __syncthreads();
        const int row0 = tile * TILE;
        if (MODE == 0) {
            for (int i = threadIdx.x; i < NR * TILE; i += NT) {
                const int n = i / TILE, j = i - n * TILE, row = row0 + j;
                if (row >= a.rows) continue;
                if (a.out_bf16) ((uint16_t*)a.y)[(size_t)n * a.ystride + row] = f2bf(tout[n][j]);
                else ((float*)a.y)[(size_t)n * a.ystride + row] = tout[n][j];
            }
        } else if (threadIdx.x < NR) {
            const int n = threadIdx.x;
            for (int j = 0; j < TILE; ++j) {
                const int row = row0 + j;
                const float v = tout[n][j];
                if (row < a.rows && finitef(v)) am_merge(bv[0], bi[0], v, (uint32_t)row);
            }
        }
        __syncthreads();
        if (next < ntiles) {
#pragma unroll
            for (int r = 0; r < RPW; ++r)
#pragma unroll
                for (int t = 0; t < NSTEP; ++t) wv[r][t] = wn[r][t];
        }
    }
    if (MODE == 1 && threadIdx.x < NR) {
        a.pval[(size_t)threadIdx.x * a.pstride + blockIdx.x] = bv[0];
        a.pidx[(size_t)threadIdx.x * a.pstride + blockIdx.x] = bi[0];
    }
    (void)bvs; (void)bis;
}

template <int NR, int MODE>
static int gemv_k(const GemvArgs& a, hipStream_t s, int* nb) {
    const int ns = (a.K + 511) / 512;
    constexpr int RPW = 2, TILE = 4 * RPW;
    const int ntiles = (a.rows + TILE - 1) / TILE;
    int grid = num_cus() * 4;
    if (MODE == 1 && grid > a.pstride) grid = a.pstride;
    if (grid > ntiles) grid = ntiles;
    if (grid < 1) grid = 1;
    if (nb) *nb = grid;
#define Q27X_G(NS) hipLaunchKernelGGL((k_gemv<NR, NS, RPW, MODE>), dim3(grid), dim3(256), 0, s, a)
    switch (ns) {
        case 1: Q27X_G(1); break;
        case 2: Q27X_G(2); break;
        case 4: Q27X_G(4); break;
        case 10: Q27X_G(10); break;
        default: return -2;
    }
#undef Q27X_G
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

int launch_gemv(const GemvArgs& a, int argmax_mode, int nr, int* nblocks_out, hipStream_t s) {
    if (!a.W || !a.x || a.rows < 1 || a.K < 8 || (a.K & 7) || nr < 1 || nr > kMaxRows) {
        set_error("gemv: bad arguments (rows=%d K=%d nr=%d)", a.rows, a.K, nr);
        return Q27X_E_ARG;
    }
    if (nr > 4) {   // instantiated for <= 4 rows (LDS stage): two launches
        GemvArgs b = a;
        int nb0 = 0, nb1 = 0;
        int rc = launch_gemv(b, argmax_mode, 4, &nb0, s);
        if (rc) return rc;
        b.x = a.x + (size_t)4 * a.xst;
        if (argmax_mode) { b.pval = a.pval + (size_t)4 * a.pstride; b.pidx = a.pidx + (size_t)4 * a.pstride; }
        else b.y = (char*)a.y + (size_t)4 * a.ystride * (a.out_bf16 ? 2 : 4);
        rc = launch_gemv(b, argmax_mode, nr - 4, &nb1, s);
        if (nblocks_out) *nblocks_out = nb0;
        return rc;
    }
    int rc = -2;
#define Q27X_GN(N) (argmax_mode ? gemv_k<N, 1>(a, s, nblocks_out) : gemv_k<N, 0>(a, s, nblocks_out))
    switch (nr) {
        case 1: rc = Q27X_GN(1); break;
        case 2: rc = Q27X_GN(2); break;
        case 3: rc = Q27X_GN(3); break;
        case 4: rc = Q27X_GN(4); break;
        default: rc = -2; break;
    }
#undef Q27X_GN
    if (rc == -2) { set_error("gemv: no kernel for K=%d nr=%d", a.K, nr); return Q27X_E_SHAPE; }
    return rc;
}

// ---------------------------------------------------------------- argmax
__global__ __launch_bounds__(256) void k_argmax_final(const float* __restrict__ pval, const uint32_t* __restrict__ pidx,
                                                      int pstride, int nblocks, int32_t* __restrict__ idx,
                                                      float* __restrict__ val, const int* stop) {
    if (stop && *stop) return;
    const int n = blockIdx.x;
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    float bv = -__builtin_huge_valf();
    uint32_t bi = 0xFFFFFFFFu;
    for (int i = threadIdx.x; i < nblocks; i += 256) {
        const uint32_t ii = pidx[(size_t)n * pstride + i];
        if (ii != 0xFFFFFFFFu) am_merge(bv, bi, pval[(size_t)n * pstride + i], ii);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
        if (oi != 0xFFFFFFFFu) am_merge(bv, bi, ov, oi);
    }
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 0; w < 4; ++w) if (si[w] != 0xFFFFFFFFu) am_merge(bv, bi, sv[w], si[w]);
        const bool none = (bi == 0xFFFFFFFFu);
        idx[n] = none ? 0 : (int32_t)bi;
        if (val) val[n] = none ? -__builtin_huge_valf() : bv;
    }
}
int launch_argmax_final(const float* pval, const uint32_t* pidx, int pstride, int nblocks, int nr,
                        int32_t* idx, float* val, const int* stop, hipStream_t s) {
    hipLaunchKernelGGL(k_argmax_final, dim3(nr), dim3(256), 0, s, pval, pidx, pstride, nblocks, idx, val, stop);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

__global__ __launch_bounds__(256) void k_argmax_part(const float* __restrict__ logits, int n, int ld,
                                                     float* __restrict__ pval, uint32_t* __restrict__ pidx, int pstride) {
    const int r = blockIdx.y;
    const float* p = logits + (size_t)r * ld;
    float bv = -__builtin_huge_valf();
    uint32_t bi = 0xFFFFFFFFu;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const float v = p[i];
        if (finitef(v)) am_merge(bv, bi, v, (uint32_t)i);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
        if (oi != 0xFFFFFFFFu) am_merge(bv, bi, ov, oi);
    }
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 0; w < 4; ++w) if (si[w] != 0xFFFFFFFFu) am_merge(bv, bi, sv[w], si[w]);
        pval[(size_t)r * pstride + blockIdx.x] = bv;
        pidx[(size_t)r * pstride + blockIdx.x] = bi;
    }
}
// module-static partials of the kernel-tier argmax (as the reference's g_q27_am_val/idx arena,
// src/q27_elem.hip:221-222): 8 rows x 64 blocks
__device__ float g_am_val[kMaxRows * 64];
__device__ uint32_t g_am_idx[kMaxRows * 64];
int argmax_scratch(float** pv, uint32_t** pi) {
    Q27X_HIP(hipGetSymbolAddress((void**)pv, HIP_SYMBOL(g_am_val)));
    Q27X_HIP(hipGetSymbolAddress((void**)pi, HIP_SYMBOL(g_am_idx)));
    return Q27X_OK;
}
int launch_argmax_rows(const float* logits, int n, int ld, int nr, int32_t* idx, float* val, float* pval,
                       uint32_t* pidx, hipStream_t s) {
    const int nb = 64;
    hipLaunchKernelGGL(k_argmax_part, dim3(nb, nr), dim3(256), 0, s, logits, n, ld, pval, pidx, nb);
    Q27X_HIP(hipGetLastError());
    return launch_argmax_final(pval, pidx, nb, nb, nr, idx, val, nullptr, s);
}

}  // namespace q27x

// ---------------------------------------------------------------- C ABI (kernel tier)
using namespace q27x;
extern "C" int q27x_proj_rows(const q27x_i8g_t* w, const int8_t* xq, int xstride, const float* xs, void* y,
                              int ystride, int out_bf16, const void* res, int res_bf16, int rstride, float rs,
                              int nr, q27x_stream_t s) {
    if (!w || !y) { set_error("q27x_proj_rows: null argument"); return Q27X_E_ARG; }
    ProjArgs a{};
    a.W = w->w; a.WS = w->s; a.rows = w->rows; a.K = w->K; a.alpha = w->alpha;
    a.xq = xq; a.xst = xstride; a.xs = xs;
    a.y = y; a.ystride = ystride; a.out_bf16 = out_bf16 ? 1 : 0;
    a.res = res; a.res_bf16 = res_bf16 ? 1 : 0; a.rstride = rstride; a.rs = rs;
    return launch_proj(a, EPI_STORE, nr, (hipStream_t)s);
}

extern "C" int q27x_proj_partials(const q27x_i8g_t* w, const int8_t* xq, int xstride, int32_t* part, int nr,
                                  q27x_stream_t s) {
    if (!w || !w->w || !xq || !part || nr < 1 || nr > kMaxRows || (w->K & 15)) {
        set_error("q27x_proj_partials: bad arguments");
        return Q27X_E_ARG;
    }
    hipLaunchKernelGGL(k_proj_partials, dim3(1024), dim3(256), 0, (hipStream_t)s, w->w, w->rows, w->K, xq, xstride,
                       part, nr);
    Q27X_HIP(hipGetLastError());
    return Q27X_OK;
}

extern "C" int q27x_bf16_gemv_rows(const uint16_t* w, int rows, int K, const uint16_t* x, int xstride, void* y,
                                   int ystride, int out_bf16, int nr, q27x_stream_t s) {
    GemvArgs a{};
    a.W = w; a.rows = rows; a.K = K; a.x = x; a.xst = xstride; a.y = y; a.ystride = ystride;
    a.out_bf16 = out_bf16 ? 1 : 0;
    if (!y) { set_error("q27x_bf16_gemv_rows: null output"); return Q27X_E_ARG; }
    return launch_gemv(a, 0, nr, nullptr, (hipStream_t)s);
}
