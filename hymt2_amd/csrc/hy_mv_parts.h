// Device building blocks of the single-token matvec, shared by the decode matvec (k_mv1) and the
// fused qkv + attention kernel: the Q8_K quantizer of two blocks per wavefront, the activation
// and weight segments of one lane, and the exact fp32 block term of one segment (the
// reference's scalar arithmetic: src/kernels.c:128-165 quantize_q8k, :565-581 panel, :808-877
// Q6_K / Q4_K).
#pragma once

#include <type_traits>

#include "hy_kernels.h"

namespace hy {

namespace {

// One lane's share of the Q8_K activation for one weight segment position.
struct ActSeg {
    int4 q0, q1, q2, q3;  // PANEL: qp rows l = 0..3; Q4K: low / high nibble qs; Q6K: groups j1 / j2
    int aux;              // Q4K: bsums[2 sub] + bsums[2 sub + 1]; Q6K: bsums[j1] | bsums[j2] << 16
    float d;
    int sum;
};

// Row (16-lane) reductions: every lane of the row receives the result.
__device__ __forceinline__ uint32_t row_max_u(uint32_t v) {
    int x = (int)v;
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP1>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP2>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_HMIRROR>(x));
    x = (int)max((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_MIRROR>(x));
    return (uint32_t)x;
}
__device__ __forceinline__ uint32_t row_min_u(uint32_t v) {
    int x = (int)v;
    x = (int)min((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP1>(x));
    x = (int)min((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_QSWAP2>(x));
    x = (int)min((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_HMIRROR>(x));
    x = (int)min((uint32_t)x, (uint32_t)hy_dpp<HY_DPP_MIRROR>(x));
    return (uint32_t)x;
}
// Q8_K of two 256-element blocks (quantize_q8k, src/kernels.c:128-165) held 8 consecutive
// elements per lane: lanes 0..31 hold dst[0]'s elements 8l..8l+7, lanes 32..63 dst[1]'s.
// The block's signed maximum stays in vector registers (a ballot and readlanes would round-trip
// through scalar ones): two row reductions and row-pair swaps, run together, of the keys
// |x| bits << 1 | sign and |x| bits << 1 | !sign give the maximum magnitude (as the unsigned
// integers order |x| bits) and tell whether it occurs with one sign only, which then is the
// first occurrence's. Only a block holding both +max and -max looks for its first occurrence
// (a third reduction, over keys 2 * index + sign of the lanes holding the magnitude).
__device__ inline void q8k_quantize_halves(const float (&e)[8], HyQ8K* dst, int lane) {
    const int hl = lane >> 5, jl = lane & 31;
    uint32_t kn[8], kp[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t u = hy_fbits(e[i]);
        kn[i] = u << 1 | u >> 31;        // ties of magnitude: the negative one is larger
        kp[i] = u << 1 | (~u >> 31);     // ties of magnitude: the positive one is larger
    }
    uint32_t mn = max(max(max(kn[0], kn[1]), max(kn[2], kn[3])), max(max(kn[4], kn[5]), max(kn[6], kn[7])));
    uint32_t mp = max(max(max(kp[0], kp[1]), max(kp[2], kp[3])), max(max(kp[4], kp[5]), max(kp[6], kp[7])));
    uint32_t ne, no, pe, po;
    mn = row_max_u(mn);
    mp = row_max_u(mp);
    hy_row_pair(mn, ne, no);
    hy_row_pair(mp, pe, po);
    mn = max(ne, no);
    mp = max(pe, po);
    const uint32_t am = mn >> 1;  // the maximum |x| bits
    uint32_t sgn = mn & 1u;       // 1 if -max occurs; then, unless +max occurs too, the sign
    if (mn & mp & 1u & (am != 0)) {  // both signs (uniform per half, so whole 16-lane rows)
        int li = 8;  // this lane's first element of magnitude am
#pragma unroll
        for (int i = 7; i >= 0; i--) li = kn[i] >> 1 == am ? i : li;
        uint32_t sg = kn[0] & 1u;
#pragma unroll
        for (int i = 1; i < 8; i++) sg = li == i ? kn[i] & 1u : sg;
        // each half holds am at least once: the smallest key is its first occurrence
        const uint32_t key = li < 8 ? ((uint32_t)(8 * jl + li) << 1 | sg) : 0xffffffffu;
        uint32_t ke, ko;
        hy_row_pair(row_min_u(key), ke, ko);
        sgn = min(ke, ko) & 1u;
    }
    const float vmax = hy_bitsf(am | sgn << 31);
    const bool zero = am == 0;
    const float iscale = zero ? 0.f : -127.f / vmax;
    const float dq = zero ? 0.f : 1.f / iscale;  // the block's d, off the path of the stores below
    int q[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = (int)__builtin_rintf(iscale * e[i]);
        q[i] = r > 127 ? 127 : (r < -127 ? -127 : r);
    }
    const int s8 = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
    const int s16 = s8 + hy_dpp<HY_DPP_QSWAP1>(s8);  // lanes 2k, 2k+1 hold one 16-element group
    uint32_t te, to;
    hy_row_pair((uint32_t)hy_group_sum<16>(s8), te, to);
    const int total = (int)(te + to);
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
    // unconditional stores, several lanes writing the same value to one address: lanes 2k and
    // 2k + 1 hold the same 16-element sum, every lane of a half the same d and sum
    y->bsums[jl >> 1] = (int16_t)s16;
    dw[296 / 4 + min(jl, 5)] = 0;
    y->d = dq;
    y->sum = total;
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

// The panel segment's exact int32 block dot enc (reduced over the block's four lanes), and the
// fp32 term made from it (src/kernels.c:576): mv1_term for KIND_PANEL in two steps, so that the
// dot can run before the activation's d and sum are final.
// Field l of a panel byte is taken in place (w & 3 << 2l: the code times 4^l, at most 48 for
// l <= 2, a non-negative int8) or, for l = 3, shifted down to the l = 2 position; the dots of
// each scale run as their own chain and the exact multiples are shifted back at the end.
__device__ __forceinline__ int mv1_panel_enc(const WSeg& S, const ActSeg& A) {
    const uint32_t w4[4] = {S.a.x, S.a.y, S.a.z, S.a.w};
    const int qa[4][4] = {{A.q0.x, A.q0.y, A.q0.z, A.q0.w}, {A.q1.x, A.q1.y, A.q1.z, A.q1.w},
                          {A.q2.x, A.q2.y, A.q2.z, A.q2.w}, {A.q3.x, A.q3.y, A.q3.z, A.q3.w}};
    int p0 = 0, p1 = 0, p2 = 0, p3 = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        p0 = hy_dot4((int)(w4[k] & 0x03030303u), qa[0][k], p0);
        p1 = hy_dot4((int)(w4[k] & 0x0C0C0C0Cu), qa[1][k], p1);
        p2 = hy_dot4((int)(w4[k] & 0x30303030u), qa[2][k], p2);
        p3 = hy_dot4((int)((w4[k] >> 2) & 0x30303030u), qa[3][k], p3);
    }
    return hy_quad_sum(p0 + (p1 >> 2) + ((p2 + p3) >> 4));
}
__device__ __forceinline__ float mv1_panel_term(const WSeg& S, int enc, float d, int sum, int pshift, int poff) {
    return hy_bitsf(S.sd) * d * (float)((enc << pshift) - poff * sum);
}

// fp32 block term of one segment, the same value in every lane of the block (the dot reduced
// over the block's lanes, the block's scales). Every lane of the block must call it (DPP group
// reductions).
template <int KIND>
__device__ __forceinline__ float mv1_term(const WSeg& S, const ActSeg& A, int sub, int pshift, int poff) {
    if (KIND == KIND_PANEL) {
        // src/kernels.c:576: ps * y.d * float((enc << shift) - off * sum)
        return mv1_panel_term(S, mv1_panel_enc(S, A), A.d, A.sum, pshift, poff);
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

}  // namespace hy
