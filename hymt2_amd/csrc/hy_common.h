// Shared device-side definitions for the gfx950 Hy-MT2 backend.
//
// Numerics contract: every kernel reproduces the reference's scalar CPU arithmetic bit for bit.
// The library is compiled with -ffp-contract=off (no fused multiply-add unless written as
// fmaf/fma), correctly rounded fp32 divide/sqrt and fp32 denormals preserved, matching the
// reference's x86-64 baseline build (src/kernels.c, src/model.c).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hy_expf.h"  // expf identical to the reference's libm expf

#define HY_QK 256
#define HY_MAX_BATCH 16  // src/internal.h:12
// Tokens per forward this backend accepts (fused_forward, matmul, the device prefill): the
// reference host sends at most HY_MAX_BATCH; a host built with a larger MAX_BATCH (128-token
// prefill chunks) may send up to this many.
#define HY_MAX_CHUNK 128

// Q8_K activation block, byte-identical to the reference's q8k_block (src/internal.h:29-41).
struct alignas(64) HyQ8K {
    int8_t qp[HY_QK];    // reordered copy: qp[l*64 + j*16 + i] = qs[{0,2,1,3}[j]*64 + l*16 + i]
    float d;
    int32_t sum;
    int16_t bsums[HY_QK / 16];
    uint8_t pad[24];
    int8_t qs[HY_QK];    // natural order
};
static_assert(sizeof(HyQ8K) == 576, "q8k_block is 576 bytes");
static_assert(__builtin_offsetof(HyQ8K, d) == 256 && __builtin_offsetof(HyQ8K, sum) == 260 &&
                  __builtin_offsetof(HyQ8K, bsums) == 264 && __builtin_offsetof(HyQ8K, qs) == 320,
              "q8k_block layout");

// ----------------------------------------------------------------------------------- bits

HY_HD inline uint32_t hy_fbits(float f) { return __builtin_bit_cast(uint32_t, f); }
HY_HD inline float hy_bitsf(uint32_t u) { return __builtin_bit_cast(float, u); }

// IEEE binary16 -> binary32 (exact, hardware conversion; pinned against the reference's
// software conversion src/kernels.c:76-98 over all 65536 inputs by the GPU tests).
__device__ inline float hy_f16(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

__device__ inline float hy_bf16(uint16_t h) { return hy_bitsf((uint32_t)h << 16); }

// Round-to-nearest-even bfloat16 (same formula as src/kernels.c:107-111).
__device__ inline uint16_t hy_to_bf16(float f) {
    uint32_t u = hy_fbits(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// ----------------------------------------------------------------------------------- lanes

// DPP row controls (gfx9 encoding): quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror. All four read a lane of the same 16-lane row, so every lane has a valid source.
#define HY_DPP_QSWAP1 0xB1
#define HY_DPP_QSWAP2 0x4E
#define HY_DPP_HMIRROR 0x141
#define HY_DPP_MIRROR 0x140

// Workgroup barrier for LDS only: waits for this wave's LDS operations, not for its global
// loads, so prefetches stay in flight across it (a __syncthreads fence would drain them).
// Forces a (kernel-argument) value into SGPRs at this point. Pinning every argument a kernel
// uses at its entry makes the compiler issue all their scalar loads in one round: argument
// fields chosen by a runtime index or read after a branch otherwise become dependent round
// trips to memory (about 0.15-0.25 us each at kernel start) before the first vector load.
template <typename T>
__device__ __forceinline__ void hy_sgpr_pin(const T& v) {
    asm volatile("" ::"s"(v));
}

// A uniform int from device memory by a scalar load, waited for on its own (lgkmcnt). Read as
// `*p` in a kernel that also stores to global memory, the compiler emits a vector load, whose
// wait covers every vector load issued before it (the counter runs in order): a kernel that
// issues its bulk loads first would then wait for all of them to learn, say, the position. The
// value must not be written by the kernel itself (the scalar cache is not coherent with vector
// stores; a kernel's start invalidates it).
__device__ __forceinline__ int hy_sload_i32(const int* p) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

// Entry i (i < 32) of hy_expf's table, for a kernel that keeps a copy in LDS (hy_expf_tab): the
// load is issued at kernel entry and the value stored to LDS before a barrier that precedes the
// first expf, so no lookup waits on global memory.
__device__ __forceinline__ uint64_t hy_exp_tab_entry(int i) {
    constexpr uint64_t T[32] = {HY_EXP2F_TABLE};
    return T[i & 31];
}

// Key of logit v at row idx for the greedy argmax of src/model.c:945-948, which starts from
// bv = logits[0] and takes row j only when logits[j] > bv: the first maximal row wins, a NaN at
// row j > 0 never wins, and a NaN at row 0 wins outright (no comparison with it is true).
__device__ inline unsigned long long argmax_key(float v, int idx) {
    uint32_t u = hy_fbits(v);
    if (u == 0x80000000u) u = 0;                       // -0 ties with +0 (first index wins)
    if ((u & 0x7fffffffu) > 0x7f800000u) return idx == 0 ? ~0ull : 0ull;
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)ord << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}


__device__ __forceinline__ void hy_lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int CTRL>
__device__ inline int hy_dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

__device__ inline int hy_quad_sum(int v) {
    v += hy_dpp<HY_DPP_QSWAP1>(v);
    v += hy_dpp<HY_DPP_QSWAP2>(v);
    return v;
}

// Sum over aligned groups of G lanes (integer, exact in any order). G <= 16 stays in DPP.
template <int G>
__device__ inline int hy_group_sum(int v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group");
    if (G >= 2) v += hy_dpp<HY_DPP_QSWAP1>(v);
    if (G >= 4) v += hy_dpp<HY_DPP_QSWAP2>(v);
    if (G >= 8) v += hy_dpp<HY_DPP_HMIRROR>(v);
    if (G >= 16) v += hy_dpp<HY_DPP_MIRROR>(v);
    return v;
}

// Both rows' values of this lane's row pair (rows 0/1 and 2/3, the two half-wavefronts):
// v_permlane16_swap of v with itself returns the even row's value and the odd row's value in
// every lane of the pair.
__device__ __forceinline__ void hy_row_pair(uint32_t v, uint32_t& even, uint32_t& odd) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    even = r[0], odd = r[1];
}
// Both halves' values at this lane's position (v_permlane32_swap of v with itself).
__device__ __forceinline__ void hy_half_pair(uint32_t v, uint32_t& lo, uint32_t& hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    lo = r[0], hi = r[1];
}

// Whole-wave reductions of an exact, order-free operation: DPP inside each 16-lane row, then the
// row pairs and the halves by the two permlane swaps, with no round trip through scalar
// registers (or LDS, as a shuffle would take). Every lane receives the result. Requires all 64
// lanes active.
template <typename Op>
__device__ __forceinline__ uint32_t hy_wave_reduce(uint32_t x, Op op) {
    x = op(x, (uint32_t)hy_dpp<HY_DPP_QSWAP1>((int)x));
    x = op(x, (uint32_t)hy_dpp<HY_DPP_QSWAP2>((int)x));
    x = op(x, (uint32_t)hy_dpp<HY_DPP_HMIRROR>((int)x));
    x = op(x, (uint32_t)hy_dpp<HY_DPP_MIRROR>((int)x));
    uint32_t a, b;
    hy_row_pair(x, a, b);
    x = op(a, b);
    hy_half_pair(x, a, b);
    return op(a, b);
}

__device__ inline int hy_wave_sum_i(int v) {
    return (int)hy_wave_reduce((uint32_t)v, [](uint32_t a, uint32_t b) { return a + b; });
}

__device__ inline uint32_t hy_wave_max_u(uint32_t v) {
    return hy_wave_reduce(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}

__device__ inline int hy_wave_min_i(int x) {
    return (int)hy_wave_reduce((uint32_t)x, [](uint32_t a, uint32_t b) { return (int)a < (int)b ? a : b; });
}

__device__ inline float hy_wave_max(float v) {
    // fmax is exact and order-free; NaN-free inputs assumed
    return __builtin_bit_cast(float, hy_wave_reduce(__builtin_bit_cast(uint32_t, v), [](uint32_t a, uint32_t b) {
        return __builtin_bit_cast(uint32_t, fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b)));
    }));
}

__device__ inline unsigned long long wave_max_u64(unsigned long long v) {
    // the same DPP row steps and permlane swaps as hy_wave_reduce, on both 32-bit halves
    uint32_t hi = (uint32_t)(v >> 32), lo = (uint32_t)v;
    auto take = [&](uint32_t h2, uint32_t l2) __attribute__((always_inline)) {
        const bool gt = h2 > hi || (h2 == hi && l2 > lo);
        hi = gt ? h2 : hi;
        lo = gt ? l2 : lo;
    };
    take((uint32_t)hy_dpp<HY_DPP_QSWAP1>((int)hi), (uint32_t)hy_dpp<HY_DPP_QSWAP1>((int)lo));
    take((uint32_t)hy_dpp<HY_DPP_QSWAP2>((int)hi), (uint32_t)hy_dpp<HY_DPP_QSWAP2>((int)lo));
    take((uint32_t)hy_dpp<HY_DPP_HMIRROR>((int)hi), (uint32_t)hy_dpp<HY_DPP_HMIRROR>((int)lo));
    take((uint32_t)hy_dpp<HY_DPP_MIRROR>((int)hi), (uint32_t)hy_dpp<HY_DPP_MIRROR>((int)lo));
    uint32_t h0, h1, l0, l1;
    hy_row_pair(hi, h0, h1);
    hy_row_pair(lo, l0, l1);
    hi = h0, lo = l0;
    take(h1, l1);
    hy_half_pair(hi, h0, h1);
    hy_half_pair(lo, l0, l1);
    hi = h0, lo = l0;
    take(h1, l1);
    return ((unsigned long long)hi << 32) | lo;
}

// The greedy argmax key of a workgroup (the maximum of every thread's key) into *slot, written by
// thread 0: one slot per workgroup, reduced by the step's finishing kernel, so no two workgroups
// write one address (same-address atomics from a whole grid serialize). Every thread calls it.
__device__ inline void hy_wg_slot_max(unsigned long long key, unsigned long long* slot) {
    __shared__ unsigned long long wk[16];
    key = wave_max_u64(key);
    const int nw = (blockDim.x + 63) >> 6;
    if ((threadIdx.x & 63) == 0) wk[threadIdx.x >> 6] = key;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < nw; w++) key = wk[w] > key ? wk[w] : key;
        *slot = key;
    }
}

// 4 bytes of 2-bit codes in field l of each byte of w, as 4 unsigned bytes 0..3.
__device__ inline int hy_field(uint32_t w, int l) { return (int)((w >> (2 * l)) & 0x03030303u); }

__device__ inline int hy_dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Sequential fp32 sum p[0] + p[1] + ... + p[n-1] in index order, computed by one whole
// wavefront (all 64 lanes active; the result is wave-uniform). p may be LDS or global, 16-byte
// aligned. Lane L loads elements [32L, 32L + 32) of each 2048-element round into registers;
// then, for L = 0, 1, ..., lane L adds its 32 registers in order to the running sum that lane
// L - 1 finished, moved one lane on by DPP (hy_lane_chain32). Only lane L's additions matter
// in step L, so the result is exactly the one-lane sequential sum, while the chain runs from
// registers at the add latency with no round trip through a scalar register (a readlane
// broadcast per step measured slower). Elements past n are read as +0.0f, which leaves the sum
// unchanged bit for bit because every sum taken here (squares, exponentials) is non-negative,
// so the running sum is never -0.
// Lane L's 32 values x[e0 .. e0 + 32) of a row of n (+0 past n): whole groups with 16-byte
// loads; the one lane that straddles n reads each element at an index clamped below n and
// selects +0 past it (no per-element branch: with branches the wavefront would run 32
// exec-masked loads, each waited for, whenever any lane straddles or passes the end).
__device__ inline void hy_lane_load32(const float* p, int e0, int n, float (&v)[32]) {
    if (e0 + 32 <= n) {
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const float4 q = *reinterpret_cast<const float4*>(p + e0 + i);
            v[i] = q.x;
            v[i + 1] = q.y;
            v[i + 2] = q.z;
            v[i + 3] = q.w;
        }
    } else if (e0 < n) {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = p[min(e0 + i, n - 1)];
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = e0 + i < n ? v[i] : 0.f;
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = 0.f;
    }
}

// The lane-serial chain over 32 registers per lane: step L adds lane L's 32 values, in order,
// to the running sum that lane L - 1 finished (moved one lane on by DPP wave_ror:1 and folded
// into the first add; step 0 starts from s in every lane). nl >= 1 steps, uniform. The result
// is in lane nl - 1; every lane receives it.
__device__ inline float hy_lane_chain32(float s, const float (&v)[32], int nl) {
    float t = s + v[0];
#pragma unroll
    for (int i = 1; i < 32; i++) t += v[i];
    for (int L = 1; L < nl; L++) {
        t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x13C, 0xF, 0xF, false)) +
            v[0];
#pragma unroll
        for (int i = 1; i < 32; i++) t += v[i];
    }
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), nl - 1));
}

// Up to four sequential fp32 sums in index order by one wavefront, one per 16-lane row: row r
// sums p[r * stride + 0 .. n) (rows from ROWS on repeat the last one). Lane i of a row holds
// elements [32 i, 32 i + 32) of each 512-element round, and the chain steps as in
// hy_lane_chain32 with DPP row_ror:1 (lane i takes lane i - 1 of its own row), so the four
// sums run in the same instructions and cost what one costs. A full round ends in lane 15 of
// the row and rotates into lane 0 as the next round's start. Every lane receives all the sums.
template <int ROWS>
__device__ inline void hy_row_seq_sums(const float* p, int stride, int n, int lane, float (&s)[4]) {
    static_assert(ROWS >= 1 && ROWS <= 4, "one sum per 16-lane row");
    const float* pr = p + (size_t)min(lane >> 4, ROWS - 1) * stride;
    const int e = 32 * (lane & 15);
    float c = 0.f, t = 0.f;  // c: in lane 0 of row r, row r's sum before the round
    int nl = 1;
    for (int base = 0; base < n; base += 16 * 32) {
        float v[32];
        hy_lane_load32(pr, base + e, n, v);
        nl = __builtin_amdgcn_readfirstlane(min(16, (n - base + 31) / 32));
        t = c + v[0];
#pragma unroll
        for (int i = 1; i < 32; i++) t += v[i];
        for (int L = 1; L < nl; L++) {
            t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x121, 0xF, 0xF, false)) +
                v[0];
#pragma unroll
            for (int i = 1; i < 32; i++) t += v[i];
        }
        c = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x121, 0xF, 0xF, false));
    }
#pragma unroll
    for (int r = 0; r < 4; r++) s[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), 16 * r + nl - 1));
}

__device__ inline float hy_wave_seq_sum(const float* p, int n, int lane) {
    float s = 0.f;
    for (int base = 0; base < n; base += 64 * 32) {
        float v[32];
        const int e0 = base + 32 * lane;
        hy_lane_load32(p, e0, n, v);
        s = hy_lane_chain32(s, v, __builtin_amdgcn_readfirstlane(min(64, (n - base + 31) / 32)));
    }
    return s;
}

// Sequential fp32 sum of squares x[0]*x[0] + x[1]*x[1] + ... in index order (each square
// rounded to fp32 first, as `sum += x[i] * x[i]` compiles without contraction), by one whole
// wavefront, with the lane-serial scheme of hy_wave_seq_sum. x is global or LDS, 16-byte aligned.
__device__ inline float hy_wave_seq_sq_sum(const float* x, int n, int lane) {
    float s = 0.f;
    for (int base = 0; base < n; base += 64 * 32) {
        float v[32];
        const int e0 = base + 32 * lane;
        hy_lane_load32(x, e0, n, v);
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = v[i] * v[i];  // +0 past n stays +0
        s = hy_lane_chain32(s, v, __builtin_amdgcn_readfirstlane(min(64, (n - base + 31) / 32)));
    }
    return s;
}

// ----------------------------------------------------------------------------------- scans

// Inclusive prefix sums over the 64 lanes (row_shr within 16-lane rows, then row_bcast:15 and
// row_bcast:31 across rows). The float version is used only for estimates (its rounding
// depends on the tree); the double version is exact wherever it is used below.
__device__ inline float hy_wave_incl_scan(float x) {
#define HY_SCAN_STEP(CTRL, ROWS)                                                                      \
    x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROWS, \
                                                               0xF, true))
    HY_SCAN_STEP(0x111, 0xF);
    HY_SCAN_STEP(0x112, 0xF);
    HY_SCAN_STEP(0x114, 0xF);
    HY_SCAN_STEP(0x118, 0xF);
    HY_SCAN_STEP(0x142, 0xA);
    HY_SCAN_STEP(0x143, 0xC);
#undef HY_SCAN_STEP
    return x;
}

__device__ inline double hy_wave_incl_scan_d(double x) {
#define HY_SCAN_STEP(CTRL, ROWS)                                                                  \
    do {                                                                                          \
        const uint64_t u = __builtin_bit_cast(uint64_t, x);                                       \
        const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROWS, 0xF, true); \
        const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROWS, 0xF, true); \
        x += __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);                               \
    } while (0)
    HY_SCAN_STEP(0x111, 0xF);
    HY_SCAN_STEP(0x112, 0xF);
    HY_SCAN_STEP(0x114, 0xF);
    HY_SCAN_STEP(0x118, 0xF);
    HY_SCAN_STEP(0x142, 0xA);
    HY_SCAN_STEP(0x143, 0xC);
#undef HY_SCAN_STEP
    return x;
}

__device__ inline double hy_readlane_d(double x, int l) {
    const uint64_t u = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// ----------------------------------------------------------------------------------- exact sums

// The sequential fp32 sum of squares s = (((0 + x0*x0) + x1*x1) + ...) for n <= 2048, bit for
// bit, computed by one whole wavefront faster than a chain of n dependent adds.
//
// Why it is exact: the addends a_i = x_i*x_i are >= 0, so the running sum s never decreases.
// While s and s + a stay in one binade [M, 2M) (ulp u = M * 2^-23), fl(s + a) = s + RN_u(a),
// where RN_u(a) rounds a to a multiple of u, unless a lies exactly halfway between two
// multiples of u (then the result depends on the parity of s). So on a stretch of addends
// where that holds, the sequential sum is s_start + sum of RN_u(a_i), which needs no chain.
//
// Lane L holds addends [32L, 32L+32) as two 16-addend segments. An estimate G of the running
// sum before each segment (float sums of non-negative values, relative error < 2^-19) places
// the segment in a binade; the true running sum differs from the exact real prefix sum by at
// most n * 2^-23 <= 2^-12 relative, so G is within 2^-11 of it, and a segment whose estimated
// start and end lie inside one binade with a 2^-9 margin is certain to run inside it. Such "clean" segments with no halfway
// addend contribute K = sum of RN_u(a_i) (exact in fp32: multiples of u below M). All clean
// K are summed in double prefix sums, exact because they are multiples of the smallest ulp in
// play and the binades used span at most 27 (checked). Remaining "dirty" segments (the
// first, those that cross a binade, those with a halfway addend) are added one addend at a
// time with fp32 adds, in order, with the clean contributions in between added exactly.
// All-zero segments are clean with K = 0. Non-finite sums make every segment dirty.
//
// hy_wave_load32 fetches lane L's values x[32L .. 32L+32) (zero past n); hy_wave_exact_sq_sum_v
// takes them, so a caller can issue the loads early.
__device__ inline void hy_wave_load32(const float* x, int n, int lane, float (&v)[32]) {
    hy_lane_load32(x, 32 * lane, n, v);
}

__device__ inline float hy_wave_exact_sq_sum_v(const float (&xv)[32], int lane) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = xv[i] * xv[i];
    // 1. estimates of the running sum before each segment
    float g[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        float t8[8];
#pragma unroll
        for (int i = 0; i < 8; i++) t8[i] = v[16 * q + 2 * i] + v[16 * q + 2 * i + 1];
        g[q] = ((t8[0] + t8[1]) + (t8[2] + t8[3])) + ((t8[4] + t8[5]) + (t8[6] + t8[7]));
    }
    const float gl = g[0] + g[1];
    // exclusive prefix as the inclusive scan of the values shifted one lane up (wave_shr:1;
    // lane 0 reads 0): a sum of non-negative terms only, so its relative error stays tiny
    const float est0 = hy_wave_incl_scan(
        __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, gl), 0x138, 0xF, 0xF, true)));
    const float tail = est0 + gl;
    const float total = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tail), 63));
    const int ex_total = (int)((hy_fbits(total) >> 23) & 0xffu);
    // 2. classify each segment; K = its exact contribution when clean
    bool clean[2];
    float K[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const float G = q ? est0 + g[0] : est0;
        const int ex = (int)((hy_fbits(G) >> 23) & 0xffu);
        const float M = hy_bitsf((uint32_t)ex << 23);
        const float hu = hy_bitsf((uint32_t)max(ex - 24, 1) << 23);  // u / 2
        bool ok = G > 0.f && ex >= 25 && ex <= 253 && ex >= ex_total - 27 && G >= M * 1.001953125f &&
                  G + g[q] < M * 1.99609375f;
        float k = 0.f;
        bool tie = false;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float a = v[16 * q + i];
            const float r = (M + a) - M;
            tie |= fabsf(a - r) == hu;
            k += r;
        }
        const bool zero = g[q] == 0.f;  // all addends +0 (g is a sum of non-negative values)
        clean[q] = zero || (ok && !tie);
        K[q] = zero ? 0.f : k;
    }
    // 3. exact prefix sums of the clean contributions, in addend order (position 2L + q)
    const double kd0 = clean[0] ? (double)K[0] : 0.0, kd1 = clean[1] ? (double)K[1] : 0.0;
    const double kl = kd0 + kd1;
    const double pin = hy_wave_incl_scan_d(kl);
    const double pex = pin - kl;  // before segment (L, 0); before (L, 1) is pex + kd0
    const uint64_t d0 = __builtin_amdgcn_ballot_w64(!clean[0]);
    const uint64_t d1 = __builtin_amdgcn_ballot_w64(!clean[1]);
    // 4. for each dirty segment, the clean contribution since the previous dirty one. Between
    //    two dirty segments every non-zero clean segment lies in one binade [M, 2M) (two clean
    //    neighbours in different binades would need a gap between their margins), so this sum
    //    is a multiple of that binade's ulp below M: exact as a float, and s + delta is exact.
    const uint64_t below = (1ull << lane) - 1;  // lanes < this one
    const uint64_t cb = (d0 | d1) & below;
    const int lp = cb ? 63 - __builtin_clzll(cb) : -1;  // last lane below with a dirty segment
    const bool lp_second = lp >= 0 && ((d1 >> lp) & 1);
    const int src = lp >= 0 ? lp : 0;
    const double pex_lp = __builtin_bit_cast(double, ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(__builtin_bit_cast(uint64_t, pex) >> 32), src) << 32) |
                                                         (uint32_t)__shfl((int)(uint32_t)__builtin_bit_cast(uint64_t, pex), src));
    const double kd0_lp = __builtin_bit_cast(double, ((uint64_t)(uint32_t)__shfl((int)(uint32_t)(__builtin_bit_cast(uint64_t, kd0) >> 32), src) << 32) |
                                                         (uint32_t)__shfl((int)(uint32_t)__builtin_bit_cast(uint64_t, kd0), src));
    const double prev0 = lp < 0 ? 0.0 : (lp_second ? pex_lp + kd0_lp : pex_lp);
    const float delta0 = (float)(pex - prev0);                       // before (L, 0)
    const float delta1 = ((d0 >> lane) & 1) ? 0.f : (float)((pex + kd0) - prev0);  // before (L, 1)
    // 5. compact the dirty segments, in order, into rows of LDS: row k = [delta, 16 addends] of
    //    the k-th dirty segment; lane k then holds row k (and k + 64)
    __shared__ float rows[128][20];
    const int rank0 = __builtin_popcountll(d0 & below) + __builtin_popcountll(d1 & below);
    const bool dirty0 = (d0 >> lane) & 1, dirty1 = (d1 >> lane) & 1;
    const int rank1 = rank0 + (dirty0 ? 1 : 0);
    if (dirty0) {
        rows[rank0][0] = delta0;
#pragma unroll
        for (int i = 0; i < 16; i++) rows[rank0][1 + i] = v[i];
    }
    if (dirty1) {
        rows[rank1][0] = delta1;
#pragma unroll
        for (int i = 0; i < 16; i++) rows[rank1][1 + i] = v[16 + i];
    }
    const int nd = __builtin_popcountll(d0) + __builtin_popcountll(d1);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // 6. the walk: s + delta is exact; then the segment's addends one fp32 add at a time. Lane
    //    k holds row k of a batch of 64; step k adds row k to the running sum rotated in from
    //    lane k - 1 (DPP wave_ror:1; lane 0 takes lane 63's, the previous batch's end).
    float t = 0.f;
    for (int base = 0; base < nd; base += 64) {
        float r[17];
        const int k = min(base + lane, 127);
#pragma unroll
        for (int i = 0; i < 17; i++) r[i] = rows[k][i];
        const int cnt = min(64, nd - base);
        for (int kk = 0; kk < cnt; kk++) {
            t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x13C, 0xF, 0xF,
                                                                      false)) + r[0];
#pragma unroll
            for (int i = 1; i < 17; i++) t += r[i];
        }
    }
    const float s = nd ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), (nd - 1) & 63)) : 0.f;
    // 7. the clean tail after the last dirty segment
    const double p_end = hy_readlane_d(pin, 63);
    double before_last = 0.0;
    if (d0 | d1) {
        const int l0 = d0 ? 63 - __builtin_clzll(d0) : -1;
        const int l1 = d1 ? 63 - __builtin_clzll(d1) : -1;
        const bool second = l1 >= l0;  // segment 2*l1 + 1 comes after 2*l0
        const int L = second ? l1 : l0;
        before_last = hy_readlane_d(pex, L) + (second ? hy_readlane_d(kd0, L) : 0.0);
    }
    return s + (float)(p_end - before_last);
}

__device__ inline float hy_wave_exact_sq_sum(const float* x, int n, int lane) {
    float v[32];
    hy_wave_load32(x, n, lane, v);
    return hy_wave_exact_sq_sum_v(v, lane);
}

// ----------------------------------------------------------------------------------- block forms

// LDS of hy_block_exact_sum8 for a workgroup of NW wavefronts.
template <int NW>
struct HyExactLdsT {
    float wtot[NW];            // estimate of each wavefront's total
    double ktot[NW];           // each wavefront's clean contributions
    int dcnt[NW];              // dirty segments of each wavefront
    double rp[128 * NW];       // dirty segments of wavefront w from 128 w: the wavefront-local
    alignas(16) float rv[128 * NW][4];  // exclusive prefix of clean contributions, and the 4 addends
};
using HyExactLds = HyExactLdsT<4>;

// The sequential fp32 sum of n = 512 * NW non-negative addends (SQ: the squares of the given
// values), the workgroup's NW wavefronts holding 8 consecutive values per lane (lane l of
// wavefront w: values 512w + 8l .. +8), bit for bit the one-lane loop. The same method as
// hy_wave_exact_sq_sum_v with two 4-addend segments per lane, the estimates and the exact prefix
// sums carried across wavefronts through LDS. The proof there holds unchanged up to n = 4096:
// the float estimates and the sequential sum stay within 2^-12 of the exact prefix sums, inside
// the 2^-9 classification margin. Every thread of the workgroup must call it; all receive the
// sum. It ends without a barrier: S must not be written again before the next workgroup barrier.
template <int NW, bool SQ>
__device__ inline float hy_block_exact_sum8(const float (&xv)[8], HyExactLdsT<NW>& S, int wave, int lane) {
    static_assert(NW >= 1 && NW <= 8, "up to 8 wavefronts (n <= 4096)");
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = SQ ? xv[i] * xv[i] : xv[i];
    const float g0 = (v[0] + v[1]) + (v[2] + v[3]);
    const float g1 = (v[4] + v[5]) + (v[6] + v[7]);
    const float g = g0 + g1;
    // 1. estimate of the running sum before this lane's values (float sums of non-negative values)
    const float estw = hy_wave_incl_scan(
        __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, g), 0x138, 0xF, 0xF, true)));
    if (lane == 63) S.wtot[wave] = estw + g;
    __syncthreads();
    float off = 0.f, total = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        if (w < wave) off += S.wtot[w];
        total += S.wtot[w];
    }
    const int ex_total = (int)((hy_fbits(total) >> 23) & 0xffu);
    // 2. classify the lane's two segments (values 0-3, 4-7)
    bool clean[2];
    float K[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const float G = q ? (off + estw) + g0 : off + estw;
        const float gq = q ? g1 : g0;
        const int ex = (int)((hy_fbits(G) >> 23) & 0xffu);
        const float M = hy_bitsf((uint32_t)ex << 23);
        const float hu = hy_bitsf((uint32_t)max(ex - 24, 1) << 23);
        const bool ok = G > 0.f && ex >= 25 && ex <= 253 && ex >= ex_total - 27 && G >= M * 1.001953125f &&
                        G + gq < M * 1.99609375f;
        float k = 0.f;
        bool tie = false;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float a = v[4 * q + i];
            const float r = (M + a) - M;
            tie |= fabsf(a - r) == hu;
            k += r;
        }
        const bool zero = gq == 0.f;
        clean[q] = zero || (ok && !tie);
        K[q] = zero ? 0.f : k;
    }
    // 3. exact prefix sums of the clean contributions within the wavefront; the dirty segments
    //    go to this wavefront's rows in LDS with their local prefix (no cross-wavefront lookup)
    const double kd0 = clean[0] ? (double)K[0] : 0.0, kd1 = clean[1] ? (double)K[1] : 0.0;
    const double kl = kd0 + kd1;
    const double pin = hy_wave_incl_scan_d(kl);
    const double pex = pin - kl;  // exact: the same sums taken apart
    const uint64_t d0 = __builtin_amdgcn_ballot_w64(!clean[0]);
    const uint64_t d1 = __builtin_amdgcn_ballot_w64(!clean[1]);
    if (lane == 63) S.ktot[wave] = pin;
    if (lane == 0) S.dcnt[wave] = __builtin_popcountll(d0) + __builtin_popcountll(d1);
    const uint64_t below = (1ull << lane) - 1;
    const int r0 = 128 * wave + __builtin_popcountll(d0 & below) + __builtin_popcountll(d1 & below);
    if (!clean[0]) {
        S.rp[r0] = pex;
        *reinterpret_cast<float4*>(S.rv[r0]) = make_float4(v[0], v[1], v[2], v[3]);
    }
    if (!clean[1]) {
        const int r1 = r0 + (clean[0] ? 0 : 1);
        S.rp[r1] = pex + kd0;
        *reinterpret_cast<float4*>(S.rv[r1]) = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
    // 4. every wavefront: the wavefronts' offsets (one batch of LDS reads), then the dirty rows in
    //    order, global row k on lane k of a batch of 64 with its global prefix P_k. Row k adds
    //    delta_k = P_k - P_{k-1}, the clean contribution since the previous dirty segment: between
    //    two dirty segments every non-zero clean segment lies in one binade [M, 2M) (two clean
    //    neighbours in different binades would need a gap between their margins), so delta_k is a
    //    multiple of that binade's ulp below M, exact as a float, and s + delta_k is exact. Then
    //    its addends one fp32 add at a time. The walk is one chain: step k adds row k to the
    //    running sum rotated in from lane k - 1 (DPP wave_ror:1, folded into the first add; lane 0
    //    takes lane 63's, the previous batch's end), with the step count uniform (a scalar loop:
    //    a per-lane counter would put a vector compare before every branch). Every wavefront
    //    walks, so all hold the sum.
    double koff[NW];
    int roff[NW];
    double ptot = 0.0;
    int nd = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        koff[w] = ptot;
        roff[w] = nd;
        ptot += S.ktot[w];
        nd += S.dcnt[w];
    }
    nd = __builtin_amdgcn_readfirstlane(nd);
    float t = 0.f;
    double pprev = 0.0, plast = 0.0;  // P of the row before this batch; P of the last row
    for (int base = 0; base < nd; base += 64) {
        const int gk = min(base + lane, nd - 1);
        int w = 0;
#pragma unroll
        for (int q = 1; q < NW; q++)
            if (gk >= roff[q]) w = q;
        double kw = koff[0];
#pragma unroll
        for (int q = 1; q < NW; q++)
            if (w == q) kw = koff[q];
        const int r = 128 * w + (gk - roff[w]);
        const double P = S.rp[r] + kw;
        const float4 a = *reinterpret_cast<const float4*>(S.rv[r]);
        // P_{k-1}: lane k - 1's (wave_shr:1; lane 0 gets the previous batch's last)
        const uint64_t pu = __builtin_bit_cast(uint64_t, P);
        const uint32_t plo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)pu, 0x138, 0xF, 0xF, true);
        const uint32_t phi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(pu >> 32), 0x138, 0xF, 0xF, true);
        const double pm = lane ? __builtin_bit_cast(double, ((uint64_t)phi << 32) | plo) : pprev;
        const float delta = (float)(P - pm);
        const int cnt = __builtin_amdgcn_readfirstlane(min(64, nd - base));
        for (int kk = 0; kk < cnt; kk++) {
            t = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x13C, 0xF,
                                                                      0xF, false)) + delta;
            t += a.x;
            t += a.y;
            t += a.z;
            t += a.w;
        }
        pprev = hy_readlane_d(P, 63);
        plast = hy_readlane_d(P, cnt - 1);
    }
    const float s = nd ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), (nd - 1) & 63)) : 0.f;
    // 5. the clean tail after the last dirty segment (one binade, as above)
    return s + (float)(ptot - plast);
}

// The RMSNorm form: the sequential sum of squares of 512 * NW values.
template <int NW>
__device__ inline float hy_block_exact_sq_sum8(const float (&xv)[8], HyExactLdsT<NW>& S, int wave, int lane) {
    return hy_block_exact_sum8<NW, true>(xv, S, wave, lane);
}
