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

// Whole-wave reductions: DPP inside each 16-lane row, then the four row results through
// readlane. The result is wave-uniform. Requires all 64 lanes active.
__device__ inline int hy_wave_sum_i(int v) {
    v = hy_group_sum<16>(v);
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
           __builtin_amdgcn_readlane(v, 48);
}

__device__ inline uint32_t hy_wave_max_u(uint32_t v) {
    int x = (int)v;
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP1>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP2>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_HMIRROR>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_MIRROR>(x));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane(x, 0), b = (uint32_t)__builtin_amdgcn_readlane(x, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane(x, 32), d = (uint32_t)__builtin_amdgcn_readlane(x, 48);
    return max(max(a, b), max(c, d));
}

__device__ inline int hy_wave_min_i(int x) {
    x = min(x, hy_dpp<HY_DPP_QSWAP1>(x));
    x = min(x, hy_dpp<HY_DPP_QSWAP2>(x));
    x = min(x, hy_dpp<HY_DPP_HMIRROR>(x));
    x = min(x, hy_dpp<HY_DPP_MIRROR>(x));
    const int a = __builtin_amdgcn_readlane(x, 0), b = __builtin_amdgcn_readlane(x, 16);
    const int c = __builtin_amdgcn_readlane(x, 32), d = __builtin_amdgcn_readlane(x, 48);
    return min(min(a, b), min(c, d));
}

__device__ inline float hy_wave_max(float v) {
    // fmax is exact and order-free; NaN-free inputs assumed
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// 4 bytes of 2-bit codes in field l of each byte of w, as 4 unsigned bytes 0..3.
__device__ inline int hy_field(uint32_t w, int l) { return (int)((w >> (2 * l)) & 0x03030303u); }

__device__ inline int hy_dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Sequential fp32 sum p[0] + p[1] + ... + p[n-1] in index order, computed by one whole
// wavefront (all 64 lanes active; the result is wave-uniform). p may be LDS or global, 16-byte
// aligned. Lane L loads elements [32L, 32L + 32) of each 2048-element round into registers;
// then, for L = 0, 1, ..., every lane adds its 32 registers in order to the running sum and
// the running sum of lane L is broadcast to all lanes (readlane). Only lane L's additions
// matter in step L, so the result is exactly the one-lane sequential sum, while the chain runs
// from registers at the add latency. Elements past n are read as +0.0f, which leaves the sum
// unchanged bit for bit because every sum taken here (squares, exponentials) is non-negative,
// so the running sum is never -0.
__device__ inline float hy_wave_seq_sum(const float* p, int n, int lane) {
    float s = 0.f;
    for (int base = 0; base < n; base += 64 * 32) {
        float v[32];
        const int e0 = base + 32 * lane;
        if (e0 + 32 <= n) {
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const float4 q = *reinterpret_cast<const float4*>(p + e0 + i);
                v[i] = q.x;
                v[i + 1] = q.y;
                v[i + 2] = q.z;
                v[i + 3] = q.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = e0 + i < n ? p[e0 + i] : 0.f;
        }
        const int nl = min(64, (n - base + 31) / 32);
        for (int L = 0; L < nl; L++) {
            float t = s;
#pragma unroll
            for (int i = 0; i < 32; i++) t += v[i];
            s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), L));
        }
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
        if (e0 + 32 <= n) {
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const float4 q = *reinterpret_cast<const float4*>(x + e0 + i);
                v[i] = q.x * q.x;
                v[i + 1] = q.y * q.y;
                v[i + 2] = q.z * q.z;
                v[i + 3] = q.w * q.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) v[i] = e0 + i < n ? x[e0 + i] * x[e0 + i] : 0.f;
        }
        const int nl = min(64, (n - base + 31) / 32);
        for (int L = 0; L < nl; L++) {
            float t = s;
#pragma unroll
            for (int i = 0; i < 32; i++) t += v[i];
            s = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), L));
        }
    }
    return s;
}
