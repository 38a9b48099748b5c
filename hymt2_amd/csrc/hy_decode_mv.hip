// Single-token matvec of the fused decode step (nt = 1), gfx950.
//
// Work layout: 256-thread workgroups, one weight row per half-wavefront per iteration, ITERS
// iterations per wave, so a workgroup covers 8 * ITERS rows (4 * ITERS gate/up pairs) and a
// launch has a few hundred workgroups. Lane j of a half-wavefront owns the 16-byte weight
// segments j, j + 32, ... of every row it visits; those always meet the same Q8_K activation
// values, which therefore live in registers, loaded once. Every weight load of the thread is
// issued before the prologue (RMSNorm + Q8_K, or Q8_K alone), so HBM streams while the
// prologue's sequential sum runs. Per block, the lanes of one block reduce their exact int32
// partial dots with DPP; the fp32 block terms go to LDS and each row is then summed in block
// order by one lane, which also applies the epilogue (store, residual add, or SwiGLU of a
// gate/up pair). The arithmetic is the reference's scalar path (src/kernels.c:565-581 panel,
// :808-877 Q6_K / Q4_K, src/model.c:719-739 RMSNorm, :865-876 residuals and SwiGLU).
#include <type_traits>

#include "hy_kernels.h"

namespace hy {

namespace {

constexpr int kMv1Threads = 256;
constexpr int kMv1Waves = kMv1Threads / 64;
constexpr int kMv1MaxWgs = 512;

// One lane's share of the Q8_K activation for one weight segment position.
struct ActSeg {
    int4 q0, q1, q2, q3;  // PANEL: qp rows l = 0..3; Q4K: low / high nibble qs; Q6K: groups j1 / j2
    int aux;              // Q4K: bsums[2 sub] + bsums[2 sub + 1]; Q6K: bsums[j1] | bsums[j2] << 16
    float d;
    int sum;
};

// Q8_K of QB 256-element blocks at once (quantize_q8k, src/kernels.c:128-165): lane l holds
// elements 4l..4l+3 of each block and block q goes to dst[q]. Branch-free, so the QB
// independent wave reductions interleave. An all-zero block gives an all-zero record.
template <int QB>
__device__ inline void q8k_quantize_lanes(const float (&e)[QB][4], HyQ8K* dst, int lane) {
#pragma unroll
    for (int q = 0; q < QB; q++) {
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) m = max(m, hy_fbits(e[q][i]) & 0x7fffffffu);
        const uint32_t am = hy_wave_max_u(m);
        int f = 256;
#pragma unroll
        for (int i = 3; i >= 0; i--)
            if ((hy_fbits(e[q][i]) & 0x7fffffffu) == am) f = 4 * lane + i;
        const int first = hy_wave_min_i(f);
        const int fi = first & 3;
        const float cand = fi == 0 ? e[q][0] : (fi == 1 ? e[q][1] : (fi == 2 ? e[q][2] : e[q][3]));
        const float vmax = hy_bitsf((uint32_t)__builtin_amdgcn_readlane((int)hy_fbits(cand), first >> 2));
        const bool zero = am == 0;
        const float iscale = zero ? 0.f : -127.f / vmax;
        int qv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = (int)__builtin_rintf(iscale * e[q][i]);
            qv[i] = r > 127 ? 127 : (r < -127 ? -127 : r);
        }
        const int s4 = qv[0] + qv[1] + qv[2] + qv[3];
        const int s16 = hy_quad_sum(s4);
        const int total = hy_wave_sum_i(s4);
        const uint32_t packed = (uint32_t)(qv[0] & 0xff) | ((uint32_t)(qv[1] & 0xff) << 8) |
                                ((uint32_t)(qv[2] & 0xff) << 16) | ((uint32_t)(qv[3] & 0xff) << 24);
        uint32_t* dw = reinterpret_cast<uint32_t*>(dst + q);
        dw[320 / 4 + lane] = packed;  // qs, natural order
        // qp: element c*64 + l*16 + i at qp[l*64 + {0,2,1,3}[c]*16 + i] (src/internal.h:31-36)
        const int c = lane >> 4, l = (lane >> 2) & 3, i0 = 4 * (lane & 3);
        const int seg = (c == 1) ? 2 : (c == 2 ? 1 : c);
        dw[(l * 64 + seg * 16 + i0) / 4] = packed;
        if ((lane & 3) == 0) dst[q].bsums[lane >> 2] = (int16_t)s16;
        if (lane < 6) dw[296 / 4 + lane] = 0;
        if (lane == 0) {
            dst[q].d = zero ? 0.f : 1.f / iscale;
            dst[q].sum = total;
        }
    }
}

// Row (16-lane) reductions: every lane of the row receives the result.
__device__ __forceinline__ uint32_t row_max_u(uint32_t v) {
    int x = (int)v;
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP1>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP2>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_HMIRROR>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_MIRROR>(x));
    return (uint32_t)x;
}
__device__ __forceinline__ int row_min_i(int x) {
    x = min(x, hy_dpp<HY_DPP_QSWAP1>(x));
    x = min(x, hy_dpp<HY_DPP_QSWAP2>(x));
    x = min(x, hy_dpp<HY_DPP_HMIRROR>(x));
    x = min(x, hy_dpp<HY_DPP_MIRROR>(x));
    return x;
}
// the value of half-wavefront `hl` (rows 2hl and 2hl + 1) combined from the row results
__device__ __forceinline__ uint32_t half_max_u(uint32_t rowv, int hl) {
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)rowv, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)rowv, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)rowv, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)rowv, 48);
    return hl ? max(c, d) : max(a, b);
}
__device__ __forceinline__ int half_min_i(int rowv, int hl) {
    const int a = __builtin_amdgcn_readlane(rowv, 0), b = __builtin_amdgcn_readlane(rowv, 16);
    const int c = __builtin_amdgcn_readlane(rowv, 32), d = __builtin_amdgcn_readlane(rowv, 48);
    return hl ? min(c, d) : min(a, b);
}
__device__ __forceinline__ int half_sum_i(int rowv, int hl) {
    const int a = __builtin_amdgcn_readlane(rowv, 0), b = __builtin_amdgcn_readlane(rowv, 16);
    const int c = __builtin_amdgcn_readlane(rowv, 32), d = __builtin_amdgcn_readlane(rowv, 48);
    return hl ? c + d : a + b;
}

// Q8_K of two 256-element blocks (quantize_q8k, src/kernels.c:128-165) held 8 consecutive
// elements per lane: lanes 0..31 hold dst[0]'s elements 8l..8l+7, lanes 32..63 dst[1]'s.
__device__ inline void q8k_quantize_halves(const float (&e)[8], HyQ8K* dst, int lane) {
    const int hl = lane >> 5, jl = lane & 31;
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) m = max(m, hy_fbits(e[i]) & 0x7fffffffu);
    const uint32_t am = half_max_u(row_max_u(m), hl);
    int f = 256;
#pragma unroll
    for (int i = 7; i >= 0; i--)
        if ((hy_fbits(e[i]) & 0x7fffffffu) == am) f = 8 * jl + i;
    const int frow = row_min_i(f);
    const int first0 = half_min_i(frow, 0), first1 = half_min_i(frow, 1);
    const int fi = (hl ? first1 : first0) & 7;
    float cand = e[0];
#pragma unroll
    for (int i = 1; i < 8; i++) cand = fi == i ? e[i] : cand;
    const float vm0 = hy_bitsf((uint32_t)__builtin_amdgcn_readlane((int)hy_fbits(cand), first0 >> 3));
    const float vm1 = hy_bitsf((uint32_t)__builtin_amdgcn_readlane((int)hy_fbits(cand), 32 + (first1 >> 3)));
    const float vmax = hl ? vm1 : vm0;
    const bool zero = am == 0;
    const float iscale = zero ? 0.f : -127.f / vmax;
    int q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = (int)__builtin_rintf(iscale * e[i]);
        q[i] = r > 127 ? 127 : (r < -127 ? -127 : r);
    }
    const int s8 = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
    const int s16 = s8 + hy_dpp<HY_DPP_QSWAP1>(s8);  // lanes 2k, 2k+1 hold one 16-element group
    const int total = half_sum_i(hy_group_sum<16>(s8), hl);
    uint32_t p[2];
#pragma unroll
    for (int w = 0; w < 2; w++)
        p[w] = (uint32_t)(q[4 * w] & 0xff) | ((uint32_t)(q[4 * w + 1] & 0xff) << 8) |
               ((uint32_t)(q[4 * w + 2] & 0xff) << 16) | ((uint32_t)(q[4 * w + 3] & 0xff) << 24);
    HyQ8K* y = dst + hl;
    uint32_t* dw = reinterpret_cast<uint32_t*>(y);
    const int idx = 8 * jl;  // first element of this lane in the block
    dw[(320 + idx) / 4] = p[0];
    dw[(320 + idx) / 4 + 1] = p[1];
    // qp: element c*64 + l*16 + i at qp[l*64 + {0,2,1,3}[c]*16 + i] (src/internal.h:31-36)
    const int c = idx >> 6, l = (idx >> 4) & 3, i0 = idx & 15;
    const int seg = (c == 1) ? 2 : (c == 2 ? 1 : c);
    dw[(l * 64 + seg * 16 + i0) / 4] = p[0];
    dw[(l * 64 + seg * 16 + i0) / 4 + 1] = p[1];
    if ((jl & 1) == 0) y->bsums[jl >> 1] = (int16_t)s16;
    if (jl < 6) dw[296 / 4 + jl] = 0;
    if (jl == 0) {
        y->d = zero ? 0.f : 1.f / iscale;
        y->sum = total;
    }
}

// 6-bit scale / min j of a Q4_K header (src/kernels.c:839-842) from its words y, z, w.
__device__ __forceinline__ int q4k_scale(const uint4& hdr, int j) {
    const int lo = (int)((hdr.y >> (8 * (j & 3))) & 63u);
    const int hi = (int)(((hdr.w >> (8 * (j & 3))) & 0xFu) | (((hdr.y >> (8 * (j & 3) + 6)) & 3u) << 4));
    return j < 4 ? lo : hi;
}
__device__ __forceinline__ int q4k_min(const uint4& hdr, int j) {
    const int lo = (int)((hdr.z >> (8 * (j & 3))) & 63u);
    const int hi = (int)(((hdr.w >> (8 * (j & 3) + 4)) & 0xFu) | (((hdr.z >> (8 * (j & 3) + 6)) & 3u) << 4));
    return j < 4 ? lo : hi;
}

__device__ __forceinline__ int4 ld_i4(const int8_t* p) { return *reinterpret_cast<const int4*>(p); }

template <int SPB>
__device__ __forceinline__ ActSeg gather_act(const HyQ8K* act, int kind, int f) {
    const int b = f / SPB, sub = f % SPB;
    const HyQ8K* y = act + b;
    ActSeg A;
    A.d = y->d;
    A.sum = y->sum;
    A.aux = 0;
    if (kind == KIND_PANEL) {
        A.q0 = ld_i4(y->qp + 0 * 64 + sub * 16);
        A.q1 = ld_i4(y->qp + 1 * 64 + sub * 16);
        A.q2 = ld_i4(y->qp + 2 * 64 + sub * 16);
        A.q3 = ld_i4(y->qp + 3 * 64 + sub * 16);
    } else if (kind == KIND_Q4K) {
        const int g = sub >> 1, half = sub & 1;
        A.q0 = ld_i4(y->qs + 64 * g + 16 * half);
        A.q1 = ld_i4(y->qs + 64 * g + 32 + 16 * half);
        A.q2 = A.q3 = make_int4(0, 0, 0, 0);
        A.aux = (int)y->bsums[2 * sub] + (int)y->bsums[2 * sub + 1];
    } else {  // Q6K
        const int h = sub >> 2, qpair = (sub >> 1) & 1, lq = sub & 1;
        const int j1 = 8 * h + 2 * qpair + lq, j2 = j1 + 4;
        A.q0 = ld_i4(y->qs + 16 * j1);
        A.q1 = ld_i4(y->qs + 16 * j2);
        A.q2 = A.q3 = make_int4(0, 0, 0, 0);
        A.aux = (int)(uint16_t)y->bsums[j1] | ((int)y->bsums[j2] << 16);
    }
    return A;
}

// Weights of one segment: a = codes / qs / ql, b = Q4_K header / Q6_K qh, c = Q6_K scale pair,
// sd = panel scale or Q6_K f16 d (as bits).
struct WSeg {
    uint4 a, b;
    int c;
    uint32_t sd;
};

template <int SPB>
__device__ __forceinline__ WSeg load_wseg(int kind, const uint8_t* w, const uint8_t* w2, const int8_t* sc,
                                          const uint16_t* dh, const float* ps, int nb, int row, int f) {
    const int b = f / SPB, sub = f % SPB;
    const size_t blk = (size_t)row * nb + b;
    WSeg S;
    S.b = make_uint4(0, 0, 0, 0);
    S.c = 0;
    S.sd = 0;
    if (kind == KIND_PANEL) {
        S.a = *reinterpret_cast<const uint4*>(w + blk * 64 + sub * 16);
        S.sd = hy_fbits(ps[blk]);
    } else if (kind == KIND_Q4K) {
        const uint8_t* base = w + blk * 144;
        S.b = *reinterpret_cast<const uint4*>(base);
        S.a = *reinterpret_cast<const uint4*>(base + 16 + sub * 16);
    } else {
        const int h = sub >> 2, qpair = (sub >> 1) & 1, lq = sub & 1;
        S.a = *reinterpret_cast<const uint4*>(w + blk * 128 + 64 * h + 32 * qpair + 16 * lq);
        S.b = *reinterpret_cast<const uint4*>(w2 + blk * 64 + 32 * h + 16 * lq);
        const int j1 = 8 * h + 2 * qpair + lq;
        const int8_t* s = sc + blk * 16;
        S.c = (int)(uint8_t)s[j1] | ((int)(uint8_t)s[j1 + 4] << 8);
        S.sd = dh[blk];
    }
    return S;
}

// fp32 block term of one segment, valid in the lane with sub == 0 of each block. Every lane of
// the block must call it (DPP group reductions).
template <int KIND>
__device__ __forceinline__ float mv1_term(const WSeg& S, const ActSeg& A, int sub, int pshift, int poff) {
    if (KIND == KIND_PANEL) {
        const uint32_t w4[4] = {S.a.x, S.a.y, S.a.z, S.a.w};
        const int4 qa[4] = {A.q0, A.q1, A.q2, A.q3};
        int p = 0;
#pragma unroll
        for (int l = 0; l < 4; l++) {
            p = hy_dot4(hy_field(w4[0], l), qa[l].x, p);
            p = hy_dot4(hy_field(w4[1], l), qa[l].y, p);
            p = hy_dot4(hy_field(w4[2], l), qa[l].z, p);
            p = hy_dot4(hy_field(w4[3], l), qa[l].w, p);
        }
        const int enc = hy_quad_sum(p);
        // src/kernels.c:576: ps * y.d * float((enc << shift) - off * sum)
        return hy_bitsf(S.sd) * A.d * (float)((enc << pshift) - poff * A.sum);
    } else if (KIND == KIND_Q4K) {
        const uint32_t w4[4] = {S.a.x, S.a.y, S.a.z, S.a.w};
        int s0 = 0, s1 = 0;
        s0 = hy_dot4((int)(w4[0] & 0x0F0F0F0Fu), A.q0.x, s0);
        s0 = hy_dot4((int)(w4[1] & 0x0F0F0F0Fu), A.q0.y, s0);
        s0 = hy_dot4((int)(w4[2] & 0x0F0F0F0Fu), A.q0.z, s0);
        s0 = hy_dot4((int)(w4[3] & 0x0F0F0F0Fu), A.q0.w, s0);
        s1 = hy_dot4((int)((w4[0] >> 4) & 0x0F0F0F0Fu), A.q1.x, s1);
        s1 = hy_dot4((int)((w4[1] >> 4) & 0x0F0F0F0Fu), A.q1.y, s1);
        s1 = hy_dot4((int)((w4[2] >> 4) & 0x0F0F0F0Fu), A.q1.z, s1);
        s1 = hy_dot4((int)((w4[3] >> 4) & 0x0F0F0F0Fu), A.q1.w, s1);
        const int g = sub >> 1;
        const int si = q4k_scale(S.b, 2 * g) * s0 + q4k_scale(S.b, 2 * g + 1) * s1;
        const int sm = q4k_min(S.b, sub) * A.aux;
        const int sumi = hy_group_sum<8>(si);
        const int summ = hy_group_sum<8>(sm);
        const float d = hy_f16((uint16_t)(S.b.x & 0xffffu));
        const float dmin = hy_f16((uint16_t)(S.b.x >> 16));
        // src/kernels.c:875: y.d * (d * float(sumi) - dmin * float(summ))
        return A.d * (d * (float)sumi - dmin * (float)summ);
    } else {  // Q6K
        const int qpair = (sub >> 1) & 1;
        const uint32_t wl[4] = {S.a.x, S.a.y, S.a.z, S.a.w};
        const uint32_t wh[4] = {S.b.x, S.b.y, S.b.z, S.b.w};
        const int q1a[4] = {A.q0.x, A.q0.y, A.q0.z, A.q0.w};
        const int q2a[4] = {A.q1.x, A.q1.y, A.q1.z, A.q1.w};
        int d1 = 0, d2 = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = (wl[i] & 0x0F0F0F0Fu) | (((wh[i] >> (2 * qpair)) & 0x03030303u) << 4);
            const uint32_t hi = ((wl[i] >> 4) & 0x0F0F0F0Fu) | (((wh[i] >> (2 * qpair + 4)) & 0x03030303u) << 4);
            d1 = hy_dot4((int)lo, q1a[i], d1);
            d2 = hy_dot4((int)hi, q2a[i], d2);
        }
        const int sc1 = (int)(int8_t)(S.c & 0xff), sc2 = (int)(int8_t)((S.c >> 8) & 0xff);
        const int bs1 = (int)(int16_t)(A.aux & 0xffff), bs2 = A.aux >> 16;
        const int acc = sc1 * (d1 - 32 * bs1) + sc2 * (d2 - 32 * bs2);
        const int tot = hy_group_sum<8>(acc);
        // src/kernels.c:833: f16(d) * y.d * float(acc)
        return hy_f16((uint16_t)S.sd) * A.d * (float)tot;
    }
}

// Keeps the compiler from moving memory operations or other instructions across this point,
// so loads are issued in the phase order the kernel is written in (vector loads complete in
// issue order: what is issued first can be consumed first).
__device__ __forceinline__ void issue_fence() {
    __builtin_amdgcn_sched_barrier(0);
    __asm__ volatile("" ::: "memory");
}

}  // namespace

// KIND: PANEL, Q4K, Q6K, or ANY (Q4K and Q6K jobs mixed; the kind is read per workgroup).
// SPL: 16-byte segments per lane per row (the row has 32 * SPL segments).
template <int KIND, int SPL, int ITERS, int PRO>
__global__ __launch_bounds__(kMv1Threads) void k_mv1(Mv1Launch L) {
    constexpr int SPB = KIND == KIND_PANEL ? 4 : 8;  // segments per 256-weight block
    constexpr int NB = SPL * 32 / SPB;              // blocks per row
    constexpr int K = NB * HY_QK;
    constexpr int RPW = 2 * ITERS;                  // rows per wave
    static_assert(NB % (2 * kMv1Waves) == 0, "blocks per row must split in pairs over the waves");
    __shared__ __align__(64) HyQ8K act_lds[PRO == PRO_NONE ? 1 : NB];
    __shared__ float terms[kMv1Waves][RPW][NB];
    using ExLds = typename std::conditional<PRO == PRO_NORM, HyExactLds, int>::type;  // LDS of the norm only
    __shared__ ExLds ex_lds;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hh = lane >> 5, j = lane & 31;
    const int wg = blockIdx.x;
    int jsel = 0;
    if (!L.pair) {
        if (L.njobs > 1 && wg >= L.job[1].wg_begin) jsel = 1;
        if (L.njobs > 2 && wg >= L.job[2].wg_begin) jsel = 2;
    }
    // constant-index selection only (a runtime index into the argument would spill it)
    const Mv1Job J = jsel == 0 ? L.job[0] : (jsel == 1 ? L.job[1] : L.job[2]);
    const bool up = L.pair && hh;  // pair mode: half-wave 1 streams the up rows
    const int kind = KIND == KIND_ANY ? J.W.kind : KIND;
    const uint8_t* w = up ? L.job[1].W.w : J.W.w;
    const uint8_t* w2 = up ? L.job[1].W.w2 : J.W.w2;
    const int8_t* wsc = up ? L.job[1].W.sc : J.W.sc;
    const uint16_t* wdh = up ? L.job[1].W.dh : J.W.dh;
    const float* wps = up ? L.job[1].W.ps : J.W.ps;
    const int pshift = up ? L.job[1].W.pshift : J.W.pshift;
    const int poff = up ? L.job[1].W.poff : J.W.poff;
    const int n = J.W.n;
    const int row0 = (wg - J.wg_begin) * L.rows_per_wg;

    // 1. the prologue's inputs first (vector loads complete in issue order, so anything issued
    //    before the weights can be consumed without waiting for them); the residual of this
    //    lane's row as well. Wavefront w quantizes the blocks 2w*R .. 2w*R + 2R (R rounds of
    //    two blocks); a lane holds 8 consecutive elements of a block per round.
    constexpr int R = NB / (2 * kMv1Waves);
    float e[R][8], nw[R][8];
    float resid = 0.f;
    const int rrow = min(row0 + wave * RPW + lane, n - 1);  // the row this lane sums (lane < RPW)
    if (!L.pair && J.epi == EPI_ADD) resid = J.out[rrow];
    ActSeg A[SPL];
    if (PRO == PRO_NONE) {
#pragma unroll
        for (int s = 0; s < SPL; s++) A[s] = gather_act<SPB>(L.act, kind, j + 32 * s);
    }
    if (PRO != PRO_NONE) {
#pragma unroll
        for (int k = 0; k < R; k++) {
            const int off = (2 * (wave * R + k)) * HY_QK + 8 * lane;
            const float4 v0 = *reinterpret_cast<const float4*>(L.x + off);
            const float4 v1 = *reinterpret_cast<const float4*>(L.x + off + 4);
            e[k][0] = v0.x, e[k][1] = v0.y, e[k][2] = v0.z, e[k][3] = v0.w;
            e[k][4] = v1.x, e[k][5] = v1.y, e[k][6] = v1.z, e[k][7] = v1.w;
            if (PRO == PRO_NORM) {
                const float4 u0 = *reinterpret_cast<const float4*>(L.norm_w + off);
                const float4 u1 = *reinterpret_cast<const float4*>(L.norm_w + off + 4);
                nw[k][0] = u0.x, nw[k][1] = u0.y, nw[k][2] = u0.z, nw[k][3] = u0.w;
                nw[k][4] = u1.x, nw[k][5] = u1.y, nw[k][6] = u1.z, nw[k][7] = u1.w;
            }
        }
    }
    issue_fence();

    // 2. every weight load of this thread, in flight through the prologue. Rows past the end
    //    load the last row instead (unconditional loads: a conditional load would need a merge
    //    copy that waits for it); their terms are never used.
    WSeg ws[ITERS][SPL];
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int r = L.pair ? row0 + wave * ITERS + i : row0 + wave * RPW + 2 * i + hh;
        const int rl = min(r, n - 1);
#pragma unroll
        for (int s = 0; s < SPL; s++) ws[i][s] = load_wseg<SPB>(kind, w, w2, wsc, wdh, wps, NB, rl, j + 32 * s);
    }
    issue_fence();

    // 3. Q8_K activation: built in LDS by the prologue, or gathered from global memory above
    if (PRO != PRO_NONE) {
        if constexpr (PRO == PRO_NORM) {
            // RMSNorm, src/model.c:719-739: sequential sum of squares, then x * scale * w
            static_assert(R == 1, "RMSNorm prologue over 2048 values");
            const float sum = hy_block_exact_sq_sum8<kMv1Waves>(e[0], ex_lds, wave, lane);
            const float scale = 1.0f / sqrtf(sum / (float)K + L.eps);
#pragma unroll
            for (int i = 0; i < 8; i++) e[0][i] = e[0][i] * scale * nw[0][i];
        }
#pragma unroll
        for (int k = 0; k < R; k++) q8k_quantize_halves(e[k], act_lds + 2 * (wave * R + k), lane);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < SPL; s++) A[s] = gather_act<SPB>(act_lds, kind, j + 32 * s);
    }

    // 4. exact block terms -> LDS
#pragma unroll
    for (int i = 0; i < ITERS; i++) {
        const int rw = 2 * i + hh;  // row slot of this half-wave in the wave
#pragma unroll
        for (int s = 0; s < SPL; s++) {
            const int f = j + 32 * s, b = f / SPB, sub = f % SPB;
            float t;
            if (KIND == KIND_ANY) {
                t = kind == KIND_Q4K ? mv1_term<KIND_Q4K>(ws[i][s], A[s], sub, pshift, poff)
                                     : mv1_term<KIND_Q6K>(ws[i][s], A[s], sub, pshift, poff);
            } else {
                t = mv1_term<KIND>(ws[i][s], A[s], sub, pshift, poff);
            }
            if (sub == 0) terms[wave][rw][b] = t;
        }
    }
    __syncthreads();

    // 5. per-row sums in block order and the epilogue
    if (!L.pair) {
        if (lane < RPW) {
            const int r = row0 + wave * RPW + lane;
            if (r < n) {
                float acc = 0.f;
#pragma unroll
                for (int b = 0; b < NB; b++) acc += terms[wave][lane][b];
                J.out[r] = J.epi == EPI_ADD ? resid + acc : acc;  // residual: h += tmp
            }
        }
    } else if (lane < ITERS) {
        const int p = row0 + wave * ITERS + lane;
        if (p < n) {
            float g = 0.f, u = 0.f;
#pragma unroll
            for (int b = 0; b < NB; b++) g += terms[wave][2 * lane][b];
#pragma unroll
            for (int b = 0; b < NB; b++) u += terms[wave][2 * lane + 1][b];
            J.out[p] = g / (1.0f + hy_expf(-g)) * u;  // SwiGLU, src/model.c:873-876
        }
    }
}

template <int KIND, int SPL, int ITERS>
static hipError_t mv1_pro(const Mv1Launch& L, int pro, int grid, hipStream_t s) {
    constexpr int SPB = KIND == KIND_PANEL ? 4 : 8;
    constexpr int NB = SPL * 32 / SPB;
    if (pro == PRO_NONE) {
        k_mv1<KIND, SPL, ITERS, PRO_NONE><<<grid, kMv1Threads, 0, s>>>(L);
    } else if (pro == PRO_QUANT) {
        k_mv1<KIND, SPL, ITERS, PRO_QUANT><<<grid, kMv1Threads, 0, s>>>(L);
    } else {
        if constexpr (NB == 8) {  // RMSNorm prologue: hidden size 2048 of the fused step
            k_mv1<KIND, SPL, ITERS, PRO_NORM><<<grid, kMv1Threads, 0, s>>>(L);
        } else {
            return hipErrorNotSupported;
        }
    }
    return hipGetLastError();
}

template <int KIND, int SPL>
static hipError_t mv1_iters(const Mv1Launch& L, int pro, int iters, int grid, hipStream_t s) {
    if constexpr (SPL > 2) {  // K = 6144 rows: one iteration keeps the weights within the register budget
        if (iters != 1) return hipErrorNotSupported;
        return mv1_pro<KIND, SPL, 1>(L, pro, grid, s);
    } else {
        switch (iters) {
        case 1: return mv1_pro<KIND, SPL, 1>(L, pro, grid, s);
        case 2: return mv1_pro<KIND, SPL, 2>(L, pro, grid, s);
        case 3: return mv1_pro<KIND, SPL, 3>(L, pro, grid, s);
        case 4: return mv1_pro<KIND, SPL, 4>(L, pro, grid, s);
        default: return hipErrorNotSupported;
        }
    }
}

hipError_t launch_mv1(Mv1Launch& L, int pro, hipStream_t s) {
    if (L.njobs < 1 || L.njobs > kMaxJobs || (L.pair && L.njobs != 2)) return hipErrorNotSupported;
    const int K = L.job[0].W.k;
    bool panel = false, q4 = false, q6 = false;
    for (int j = 0; j < L.njobs; j++) {
        const MvWeight& W = L.job[j].W;
        if (W.k != K || W.n < 1) return hipErrorNotSupported;
        panel |= W.kind == KIND_PANEL;
        q4 |= W.kind == KIND_Q4K;
        q6 |= W.kind == KIND_Q6K;
        if (W.kind != KIND_PANEL && W.kind != KIND_Q4K && W.kind != KIND_Q6K) return hipErrorNotSupported;
    }
    if (panel && (q4 || q6)) return hipErrorNotSupported;
    if (L.pair && (L.job[0].W.kind != L.job[1].W.kind || L.job[0].W.n != L.job[1].W.n)) return hipErrorNotSupported;
    if (K != 2048 && K != 6144) return hipErrorNotSupported;
    if (pro == PRO_NORM && K != 2048) return hipErrorNotSupported;
    if (pro != PRO_NONE && !L.x) return hipErrorInvalidValue;
    // smallest ITERS whose grid fits a few workgroups per CU
    int iters = 0, grid = 0;
    const int max_iters = K == 2048 ? 4 : 1;
    for (int it = 1; it <= max_iters; it++) {
        const int per = L.pair ? kMv1Waves * it : kMv1Waves * 2 * it;
        int g = 0;
        for (int j = 0; j < (L.pair ? 1 : L.njobs); j++) {
            L.job[j].wg_begin = g;
            g += (L.job[j].W.n + per - 1) / per;
        }
        if (L.pair) L.job[1].wg_begin = 0;
        iters = it;
        grid = g;
        L.rows_per_wg = per;
        if (g <= kMv1MaxWgs) break;
    }
    L.K = K;
    const int kind = panel ? KIND_PANEL : (q4 && q6 ? KIND_ANY : (q4 ? KIND_Q4K : KIND_Q6K));
    if (kind == KIND_PANEL) {
        return K == 2048 ? mv1_iters<KIND_PANEL, 1>(L, pro, iters, grid, s) : mv1_iters<KIND_PANEL, 3>(L, pro, iters, grid, s);
    }
    if (kind == KIND_Q4K) {
        return K == 2048 ? mv1_iters<KIND_Q4K, 2>(L, pro, iters, grid, s) : mv1_iters<KIND_Q4K, 6>(L, pro, iters, grid, s);
    }
    if (kind == KIND_Q6K) {
        return K == 2048 ? mv1_iters<KIND_Q6K, 2>(L, pro, iters, grid, s) : mv1_iters<KIND_Q6K, 6>(L, pro, iters, grid, s);
    }
    return K == 2048 ? mv1_iters<KIND_ANY, 2>(L, pro, iters, grid, s) : mv1_iters<KIND_ANY, 6>(L, pro, iters, grid, s);
}

}  // namespace hy
