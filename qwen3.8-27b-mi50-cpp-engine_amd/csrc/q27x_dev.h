// q27x_dev.h -- device helpers shared by the gfx950 kernels.
//
// Numerics contract: every kernel computes its floating-point results in one fixed order with
// correctly rounded IEEE operations (no FMA contraction, correctly rounded divide and sqrt,
// explicit fmaf), and the transcendentals below are built from those operations only, so the
// results are reproducible bit for bit by a host restatement of the same order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q27x {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 (include/q27.h:133-139)
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bfr(float f) { return bf2f(f2bf(f)); }   // round through bf16

// ---------------------------------------------------------------- transcendentals
// p * 2^n for p in [0.5, 2), n in [-152, 130]; one rounding at the final product.
__device__ __forceinline__ float scale2(float p, int n) {
    if (n > 127) { p = p * 0x1p127f; n -= 127; }
    if (n < -126) { p = p * 0x1p-64f; n += 64; }
    return p * __uint_as_float((uint32_t)(n + 127) << 23);
}
// e^x: Cody-Waite reduction with ln2 split in hi/lo, degree-7 Taylor polynomial (Horner, fmaf).
// Branch-free: the polynomial runs on x clamped to the finite range (x itself wherever the
// result is finite) and the special cases are selected at the end.
__device__ __forceinline__ float qexp(float xin) {
    const float x = fminf(fmaxf(xin, -103.972084045f), 88.7228393555f);
    const float kf = rintf(x * 1.44269502163f);
    float r = __builtin_fmaf(kf, -0.693145751953125f, x);
    r = __builtin_fmaf(kf, -1.42860682e-06f, r);
    float p = 1.98412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333377e-3f);
    p = __builtin_fmaf(p, r, 4.16666679e-2f);
    p = __builtin_fmaf(p, r, 1.66666672e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float v = scale2(p, (int)kf);
    return (xin != xin) ? xin : (xin > 88.7228393555f) ? __builtin_huge_valf() : (xin < -103.972084045f) ? 0.0f : v;
}
// 2^x = 2^k * e^(r ln2), x = k + r exactly. Branch-free as qexp.
__device__ __forceinline__ float qexp2(float xin) {
    const float x = fminf(fmaxf(xin, -150.0f), 128.0f);
    const float kf = rintf(x);
    const float r = x - kf;
    float p = 1.52527336e-5f;
    p = __builtin_fmaf(p, r, 1.54035304e-4f);
    p = __builtin_fmaf(p, r, 1.33335581e-3f);
    p = __builtin_fmaf(p, r, 9.61812911e-3f);
    p = __builtin_fmaf(p, r, 5.55041087e-2f);
    p = __builtin_fmaf(p, r, 2.40226507e-1f);
    p = __builtin_fmaf(p, r, 6.93147182e-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float v = scale2(p, (int)kf);
    return (xin != xin) ? xin : (xin >= 128.0f) ? __builtin_huge_valf() : (xin < -150.0f) ? 0.0f : v;
}
// log(u), finite normal u > 0: u = m 2^e, s = (m-1)/(m+1), log m = 2 atanh(s) to s^9.
__device__ __forceinline__ float qlog_pos(float u) {
    const uint32_t b = __float_as_uint(u);
    int e = (int)((b >> 23) & 0xffu) - 127;
    float m = __uint_as_float((b & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421354f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float s2 = s * s;
    float p = 0.222222224f;
    p = __builtin_fmaf(p, s2, 0.285714298f);
    p = __builtin_fmaf(p, s2, 0.400000006f);
    p = __builtin_fmaf(p, s2, 0.666666687f);
    p = p * s2;
    const float lm = __builtin_fmaf(s, p, s + s);
    const float ef = (float)e;
    return __builtin_fmaf(ef, 0.693145751953125f, __builtin_fmaf(ef, 1.42860682e-06f, lm));
}
__device__ __forceinline__ float qlog1p(float y) {
    if (y != y) return y;
    if (y == __builtin_huge_valf()) return y;
    const float u = 1.0f + y;
    if (u == 1.0f) return y;
    return qlog_pos(u) * (y / (u - 1.0f));
}
__device__ __forceinline__ float qsigmoid(float x) { return 1.0f / (1.0f + qexp(-x)); }
__device__ __forceinline__ float qsilu(float x) { return x / (1.0f + qexp(-x)); }
__device__ __forceinline__ float qsoftplus(float x) { return (x > 20.0f) ? x : qlog1p(qexp(x)); }
__device__ __forceinline__ float rsqrt_cr(float x) { return 1.0f / __builtin_sqrtf(x); }

// s_waitcnt immediate that waits until at most n (<= 63) vector-memory operations of this wave
// are outstanding and leaves the export and LDS/scalar counters alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// LDS DMA of 16 bytes per lane: lane l's 16 bytes from g land at LDS byte address lds + 16 l
// (lds wave-uniform). Issued from inline asm: with the builtin form the compiler makes every
// later LDS read of the wave wait for all of its outstanding vector-memory loads, which would
// serialize a multi-stage pipeline; here the transfer is invisible to the compiler, and the caller
// waits for it (s_waitcnt vmcnt, counting these in issue order) before it reads the destination.
// M0 carries the LDS base for the one instruction and is restored after it.
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds) {
    uint32_t save;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(save) : "s"(lds), "v"(g) : "memory");
}

// The round's stop flag (null: never stopped), read through the constant address space so it is
// a scalar load: a vector load would make the wait for it (vmcnt) also wait for every weight load
// issued before it. The flag does not change while a kernel that reads it runs.
__device__ __forceinline__ bool stopped(const int* p) {
    typedef __attribute__((address_space(4))) const int cint;
    return p && *(cint*)p;
}
// A device-resident int that no kernel writes while the reader runs (round positions, counts),
// read the same way: a scalar load whose wait does not wait for vector loads.
__device__ __forceinline__ int ld_uniform(const int* p) {
    typedef __attribute__((address_space(4))) const int cint;
    return *(cint*)p;
}

// Request every 64-byte line of a kernel's argument struct at once, at the start: the compiler
// otherwise loads each argument near its first use, and every scalar-cache miss on the argument
// segment (written once per graph, cold by the time the launch runs) is a memory round trip in
// the middle of the prologue. One scalar load per line, one wait; later reads of any argument hit
// the scalar cache.
template <typename T>
__device__ __forceinline__ void warm_args(const T& a) {
    const char* p = (const char*)&a;
#pragma unroll
    for (int off = 0; off < (int)sizeof(T); off += 64) {
        const int v = *(const int*)(p + off);
        asm volatile("" ::"s"(v));
    }
}

// ---------------------------------------------------------------- reductions
// x of lane l + N in the same 16-lane row (DPP row_shl:N, a VALU operand route instead of an LDS
// crossbar shuffle; lanes past the row's end read 0). It equals __shfl_down(x, N) in every lane l
// with l % 16 + N < 16 -- in a halving tree with offsets N <= 8, every lane whose sum is used.
template <int N>
__device__ __forceinline__ float dpp_down(float x) {
    static_assert(N >= 1 && N <= 15, "row_shl");
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xF, 0xF, true));
}
// x of lane l ^ 32 and of lane l ^ 16, by the gfx950 lane-swap instructions (VALU, no LDS
// crossbar): v_permlane32_swap on two copies of x leaves the upper half-wave's values in the lower
// lanes of the second result and the lower half's in the upper lanes of the first;
// v_permlane16_swap does the same for odd/even 16-lane rows.
__device__ __forceinline__ float xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
// One level of a shfl_down halving tree: offsets 32 and 16 cross rows (lane swaps: lane l reads
// l ^ O, which is l + O in every lane whose sum the tree uses), 8..1 by DPP.
template <int O>
__device__ __forceinline__ float down_add(float x) {
    if constexpr (O == 32) return x + xor32(x);
    else if constexpr (O == 16) return x + xor16(x);
    else return x + dpp_down<O>(x);
}
// shfl_down tree over the 64 lanes (offsets 32..1, the same pairs in the same order); the result
// is valid in lane 0.
__device__ __forceinline__ float tree64(float x) {
    x = down_add<32>(x);
    x = down_add<16>(x);
    x = down_add<8>(x);
    x = down_add<4>(x);
    x = down_add<2>(x);
    x = down_add<1>(x);
    return x;
}
// lane 0's value in every lane (a scalar read, no crossbar)
__device__ __forceinline__ float bcast0(float x) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x)));
}
// Exact max over aligned groups of `width` (a power of two <= 64) lanes, in every lane of the
// group: quads by DPP quad permutes (l ^ 1, l ^ 2), then 8 and 16 lanes by DPP half-row and row
// mirrors (each pairs the two halves of the group, which already hold their own maxima), then the
// lane swaps for 32 and 64. The max of the same values in any order is the same float.
__device__ __forceinline__ float max_xor(float x, int width) {
    if (width >= 2) x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false)));
    if (width >= 4) x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false)));
    if (width >= 8) x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false)));
    if (width >= 16) x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false)));
    if (width >= 32) x = fmaxf(x, xor16(x));
    if (width >= 64) x = fmaxf(x, xor32(x));
    return x;
}
// The same max over the 4 lanes of a quad with DPP quad permutes (a VALU operand route, no LDS
// crossbar): lane l reads lane l ^ 2 (quad_perm [2,3,0,1]), then l ^ 1 ([1,0,3,2]). The max of the
// same four values in any order is the same float.
// lane b's value of each quad of lanes, in all four lanes (b a constant after unrolling)
__device__ __forceinline__ float quad_bcast(float x, int b) {
    const int v = __float_as_int(x);
    switch (b & 3) {
        case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x00, 0xF, 0xF, false));
        case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x55, 0xF, 0xF, false));
        case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xAA, 0xF, 0xF, false));
        default: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xFF, 0xF, 0xF, false));
    }
}
__device__ __forceinline__ float max_quad(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false)));
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false)));
    return x;
}

// ---------------------------------------------------------------- int8
__device__ __forceinline__ int dot16(const uint4 w, const uint4 x) {
    // (the first product with the clamp bit, which four int8 products can never reach: that form
    // takes the zero accumulator as an inline constant, where the unclamped one becomes the
    // two-operand instruction and needs a register cleared for every chain)
    int d = __builtin_amdgcn_sdot4((int)w.x, (int)x.x, 0, true);
    d = __builtin_amdgcn_sdot4((int)w.y, (int)x.y, d, false);
    d = __builtin_amdgcn_sdot4((int)w.z, (int)x.z, d, false);
    d = __builtin_amdgcn_sdot4((int)w.w, (int)x.w, d, false);
    return d;
}
__device__ __forceinline__ int8_t qcode(float v, float inv) {
    int c = (int)rintf(v * inv);
    c = c < -127 ? -127 : (c > 127 ? 127 : c);
    return (int8_t)c;
}
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------- grid-wide hand-off
// MI355X's L2 is private to each XCD and not coherent across XCDs; an agent-scope release fence
// (__threadfence) writes back and then invalidates the issuing XCD's whole L2, which costs tens
// of microseconds when every block of a large grid does it. Instead the values that another
// block must read inside the same kernel are written with agent-scope stores (sc1: written
// through to the coherence point), every thread waits for its stores to be acknowledged before
// the block's arrival is counted, and only the reader block invalidates its L2 (acquire fence,
// one buffer_inv) before plain loads.
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint16_t* p, uint16_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_agent(unsigned* p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Arrival counting over 16 sub-counters (one 256-B line each, cnt[64 (1 + j)]) and a top counter
// cnt[0]: same-address atomics serialize (~11 ns each on MI355X), so a flat counter over 1000+
// blocks would cost more than the work it guards. Every counter is reset by its last arrival.
// Returns true in every thread of the block that arrives last; that block has passed an
// agent-scope acquire. Called by all threads of the block after their agent-scope stores.
constexpr int kArriveLines = 17;                   // counter lines of 256 B
__device__ __forceinline__ bool arrive_last(unsigned* cnt, unsigned nblocks, unsigned* s_flag) {
    __builtin_amdgcn_s_waitcnt(0);                   // this thread's stores acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned ns = nblocks < 16u ? nblocks : 16u;
        const unsigned j = blockIdx.x % ns;
        const unsigned nj = (nblocks - j + ns - 1) / ns;   // blocks counted on sub-counter j
        unsigned last = 0u;
        if (add_agent(cnt + 64 * (1 + j), 1u) == nj - 1) {
            st_agent(cnt + 64 * (1 + j), 0u);
            if (add_agent(cnt, 1u) == ns - 1) {
                st_agent(cnt, 0u);
                last = 1u;
            }
        }
        *s_flag = last;
    }
    __syncthreads();
    if (*s_flag == 0u) return false;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return true;
}

// ---------------------------------------------------------------- synthetic generator
__host__ __device__ __forceinline__ uint64_t sm64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
__host__ __device__ __forceinline__ uint64_t tensor_key(uint64_t seed, uint64_t tensor) {
    return sm64(seed ^ (tensor * 0xD6E8FEB86659FD93ull));
}
// Irwin-Hall(4) normal: sum of four 16-bit fields (exact), one subtraction (exact), one multiply.
__device__ __forceinline__ float normal_k(uint64_t key, uint64_t idx) {
    const uint64_t h = sm64(key + idx);
    const uint32_t s = (uint32_t)(h & 0xffffu) + (uint32_t)((h >> 16) & 0xffffu) +
                       (uint32_t)((h >> 32) & 0xffffu) + (uint32_t)(h >> 48);
    return ((float)s - 131070.0f) * 2.64289800e-05f;
}
__device__ __forceinline__ float uniform_k(uint64_t key, uint64_t idx) {
    const uint64_t h = sm64(key + idx);
    return (float)(uint32_t)(h >> 40) * 0x1p-24f;
}

}  // namespace q27x
