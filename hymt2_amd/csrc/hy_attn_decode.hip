// Single-token attention of the fused decode step (nt = 1), gfx950: one 512-thread workgroup
// per query head, the reference's attn_task for one position (src/model.c:767-795) after the
// per-token RoPE, q/k RMSNorm and bf16 KV store (src/model.c:836-847).
//
// Scores: one key per thread per pass of 512 positions, dot_bf16's four interleaved partial
// sums in order (src/kernels.c:1111-1121); the first pass's key rows load at kernel entry. Softmax
// (src/model.c:781-789): max (order-free), expf, the sum in position order by the 8-wavefront
// exact segmented sum (hy_block_exact_sum8), p_j = e_j * (1 / sum) formed once per position.
// Output (axpy_bf16, src/kernels.c:1122-1124): o[d] += p_j * V_j[d] in position order, as a
// pipeline over tiles of 96 positions: wavefronts 2-7 convert the V rows of tile t + 1 to fp32
// into one half of a double-buffered [j][d] LDS tile while wavefronts 0-1 (one lane per
// dimension) walk tile t in position order, each step one multiply p_j * V_j[d] (rounded to fp32,
// as the reference rounds it) and one add; one LDS-only barrier per tile, V rows loaded three
// tiles ahead. The fp32 output row goes to `ao`; the o-projection quantizes it.
#include "hy_kernels.h"

namespace hy {

namespace {

constexpr int kA1Threads = 512;
constexpr int kA1Waves = kA1Threads / 64;
constexpr int kA1Tile = 96;            // positions per product tile
constexpr int kA1Prod = kA1Threads - 128;  // producer threads (wavefronts 2-7)
constexpr int kA1Chunk = 32;           // positions per chain step (16 LDS reads of 2 products)
constexpr int kA1SerialSum = 256;      // softmax rows up to this length: the lane-serial sum
constexpr int kA1PairRow = kA1Threads / 2;  // rows up to this length: two lanes per key
static_assert(kA1SerialSum <= kA1PairRow, "the serial sum reads the pair form's padded exponentials");
constexpr int kA1ShortRow = 2 * kA1Tile;    // rows up to this length: V staged whole, direct chains

__device__ __forceinline__ void bf16x8f(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = hy_bitsf(w[i] << 16);
        f[2 * i + 1] = hy_bitsf(w[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ void a1_fence() {
    __builtin_amdgcn_sched_barrier(0);
    __asm__ volatile("" ::: "memory");
}

}  // namespace

// RoPE (NeoX, src/model.c:754-765) and RMSNorm (src/model.c:840-841) of one head row, by one
// wavefront: lane l owns elements l, l + 64, ... (RPL per lane), with its cos / sin table
// entries (c, sn) and norm weights (nw) already in registers. scr is this wavefront's LDS row.
template <int HD>
__device__ __forceinline__ void rope_norm_wave(const float (&x)[HD / 64], float* scr, const float (&c)[HD / 64],
                                               const float (&sn)[HD / 64], int half, const float (&nw)[HD / 64],
                                               float eps, int lane, float (&out)[HD / 64]) {
    constexpr int RPL = HD / 64;
    float r[RPL];
    if (RPL == 2 && half == 64) {
        // the rotation pairs elements lane and lane + 64, both held by this lane
        r[0] = x[0] * c[0] - x[RPL - 1] * sn[0];
        r[RPL - 1] = x[0] * sn[0] + x[RPL - 1] * c[0];
    } else {
#pragma unroll
        for (int i = 0; i < RPL; i++) scr[lane + 64 * i] = x[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int d = lane + 64 * i;
            r[i] = x[i];
            if (d < half) r[i] = x[i] * c[i] - scr[d + half] * sn[i];
            else if (d < 2 * half) r[i] = scr[d - half] * sn[i] + x[i] * c[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int i = 0; i < RPL; i++) scr[lane + 64 * i] = r[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float sum = hy_wave_seq_sq_sum(scr, HD, lane);
    const float scale = 1.0f / sqrtf(sum / (float)HD + eps);
#pragma unroll
    for (int i = 0; i < RPL; i++) out[i] = r[i] * scale * nw[i];
}

// dot_bf16(q, K_j) * scale with the reference's four partial sums (src/kernels.c:1111-1121).
// q is read from LDS on every call (the offset is opaque to the compiler): held in registers
// across a loop of passes it would take HD registers of its own.
template <int HD>
__device__ __forceinline__ float a1_score(const uint4 (&k)[HD / 8], const float* qn, float scale) {
    int qo = 0;
    asm volatile("" : "+v"(qo));
    qn += qo;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 8; i++) {
        float kf[8];
        bf16x8f(k[i], kf);
        const float4 qa = *reinterpret_cast<const float4*>(qn + 8 * i);
        const float4 qb = *reinterpret_cast<const float4*>(qn + 8 * i + 4);
        a0 += qa.x * kf[0];
        a1 += qa.y * kf[1];
        a2 += qa.z * kf[2];
        a3 += qa.w * kf[3];
        a0 += qb.x * kf[4];
        a1 += qb.y * kf[5];
        a2 += qb.z * kf[6];
        a3 += qb.w * kf[7];
    }
    return ((a0 + a1) + (a2 + a3)) * scale;
}

// The same score with the key split over a pair of adjacent lanes: lane parity 0 forms the
// partial sums a0, a1 (elements 4k, 4k + 1), parity 1 forms a2, a3, each in dot_bf16's order;
// the pair swaps its halves and both lanes form ((a0 + a1) + (a2 + a3)) * scale, with the
// operands in the same positions, so both hold the same bits.
template <int HD>
__device__ __forceinline__ float a1_score_pair(const uint4 (&k)[HD / 8], const float* qn, int par, float scale) {
    int qo = 0;
    asm volatile("" : "+v"(qo));
    qn += qo + 2 * par;
    float x0 = 0.f, x1 = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 8; i++) {
        const uint32_t wa = par ? k[i].y : k[i].x;  // elements 8i + 2 par, + 1
        const uint32_t wb = par ? k[i].w : k[i].z;  // elements 8i + 4 + 2 par, + 1
        const float2 qa = *reinterpret_cast<const float2*>(qn + 8 * i);
        const float2 qb = *reinterpret_cast<const float2*>(qn + 8 * i + 4);
        x0 += qa.x * hy_bitsf(wa << 16);
        x1 += qa.y * hy_bitsf(wa & 0xffff0000u);
        x0 += qb.x * hy_bitsf(wb << 16);
        x1 += qb.y * hy_bitsf(wb & 0xffff0000u);
    }
    const float own = x0 + x1;
    const float other = __builtin_bit_cast(float, hy_dpp<HY_DPP_QSWAP1>(__builtin_bit_cast(int, own)));
    return (par ? other + own : own + other) * scale;
}

template <int HD>
__device__ __forceinline__ void a1_load_key(uint4 (&k)[HD / 8], const uint16_t* K, int row) {
#pragma unroll
    for (int i = 0; i < HD / 8; i++) k[i] = *reinterpret_cast<const uint4*>(K + (size_t)row * HD + 8 * i);
}

// Producer work split: V rows in quads of 4 dimensions (8 bytes). Producer thread p
// (0 .. kA1Prod - 1) owns quad p % QPR of rows p / QPR + RSTEP k, k < IPT, of every tile: a
// wavefront's loads of one k cover whole rows (contiguous global memory), its product stores
// one contiguous run of the [j][d] tile.
template <int HD>
struct A1Split {
    static constexpr int QPR = HD / 4;                   // quads per row
    static constexpr int IPT = kA1Tile * QPR / kA1Prod;  // quads per producer thread per tile
    static constexpr int RSTEP = kA1Prod / QPR;          // rows between a thread's quads
    static_assert(kA1Prod % QPR == 0 && kA1Tile % RSTEP == 0, "whole rows per producer step");
};

// V quads of one tile for producer thread p: rows t0 + row (clamped to `last`)
template <int HD>
__device__ __forceinline__ void a1_load_v(uint2 (&v)[A1Split<HD>::IPT], const uint16_t* V, int t0, int p, int last) {
    using P = A1Split<HD>;
    const int r0 = t0 + p / P::QPR, q = p % P::QPR;
#pragma unroll
    for (int k = 0; k < P::IPT; k++)
        v[k] = *reinterpret_cast<const uint2*>(V + (size_t)min(r0 + P::RSTEP * k, last) * HD + 4 * q);
}

// o += p_j * V_j[d] in position order over the first nch chunks of 32 positions of a tile
// ([j][d] fp32 layout: lane d reads col = tile + d, two positions per LDS read; pj = the tile's
// p_j, the same for every lane). Positions past the row have V = +0 and p_j = +0, so they add
// +0, which leaves o unchanged (o is never -0: it starts at +0, and a sum of nonzero addends that
// cancels rounds to +0). The reads of the next chunk are issued before a chunk is added, and
// scheduling barriers keep them there: left to itself the compiler moves each read next to its
// use, and the chain then waits out the LDS latency at every position.
template <int HD>
__device__ __forceinline__ void a1_chain(const float* col, const float* pj, int nch, float& o) {
    static_assert(kA1Tile == 3 * kA1Chunk, "three chunks per tile");
    constexpr int C = kA1Chunk / 2;  // positions per step
    float va[C], pa[C], vb[C], pb[C];
    auto ld = [&](float (&v)[C], float (&p)[C], int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < C; i += 4) {
            const float4 q = *reinterpret_cast<const float4*>(pj + j0 + i);
            p[i] = q.x, p[i + 1] = q.y, p[i + 2] = q.z, p[i + 3] = q.w;
        }
#pragma unroll
        for (int i = 0; i < C; i++) v[i] = col[(j0 + i) * HD];
    };
    auto add = [&](const float (&v)[C], const float (&p)[C]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < C; i++) o += p[i] * v[i];
    };
    const int steps = 2 * nch;
    ld(va, pa, 0);
    for (int c = 0; c < steps; c += 2) {  // no exit inside the body: the prefetches stay where written
        ld(vb, pb, (c + 1) * C);
        __builtin_amdgcn_sched_barrier(0);
        add(va, pa);
        __builtin_amdgcn_sched_barrier(0);
        ld(va, pa, min(c + 2, 2 * (kA1Tile / kA1Chunk) - 1) * C);
        __builtin_amdgcn_sched_barrier(0);
        add(vb, pb);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// V rows of one tile as fp32 into buf[j][d] (16-byte stores) for producer thread p's quads.
// EDGE (the tile reaches the row's end): position `pos` takes this token's V row from LDS (vb,
// all read before any value is stored) and positions past the row are +0.
template <int HD, bool EDGE>
__device__ __forceinline__ void a1_stage_tile(const uint2 (&v)[A1Split<HD>::IPT], float* buf, const uint16_t* vb,
                                              int t0, int p, int pos, int n) {
    using P = A1Split<HD>;
    const int r0 = p / P::QPR, q = p % P::QPR;
    uint2 w[P::IPT];
#pragma unroll
    for (int k = 0; k < P::IPT; k++) w[k] = v[k];
    if constexpr (EDGE) {
        const uint2 b = *reinterpret_cast<const uint2*>(vb + 4 * q);
#pragma unroll
        for (int k = 0; k < P::IPT; k++) {
            const bool cur = t0 + r0 + P::RSTEP * k == pos;
            w[k] = {cur ? b.x : w[k].x, cur ? b.y : w[k].y};
        }
    }
#pragma unroll
    for (int k = 0; k < P::IPT; k++) {
        const int r = r0 + P::RSTEP * k;
        float4 x = make_float4(hy_bitsf(w[k].x << 16), hy_bitsf(w[k].x & 0xffff0000u), hy_bitsf(w[k].y << 16),
                               hy_bitsf(w[k].y & 0xffff0000u));
        if (EDGE && t0 + r >= n) x = {0.f, 0.f, 0.f, 0.f};
        *reinterpret_cast<float4*>(buf + r * HD + 4 * q) = x;
    }
}

// Short rows: V of the tile at t0 as fp32 into stage[j][d] for producer thread p's quads (rows
// below n; position `pos` from this token's V row in LDS, vb).
template <int HD>
__device__ __forceinline__ void a1_stage_v(const uint2 (&v)[A1Split<HD>::IPT], float* stage, const uint16_t* vb,
                                           int t0, int p, int pos, int n) {
    using P = A1Split<HD>;
    const int r0 = t0 + p / P::QPR, q = p % P::QPR;
    const uint2 b = *reinterpret_cast<const uint2*>(vb + 4 * q);
#pragma unroll
    for (int k = 0; k < P::IPT; k++) {
        const int r = r0 + P::RSTEP * k;
        if (r < n) {
            const uint2 w = r == pos ? b : v[k];
            *reinterpret_cast<float4*>(stage + r * HD + 4 * q) =
                make_float4(hy_bitsf(w.x << 16), hy_bitsf(w.x & 0xffff0000u), hy_bitsf(w.y << 16), hy_bitsf(w.y & 0xffff0000u));
        }
    }
}

// Short rows: o = sum_j p_j * V_j[d] in position order for lane d (col = stage + d, p_j in
// LDS). Chunks of 16 positions in two register sets: the next chunk's LDS reads are in flight
// while a chunk is added (a loop over chunk pairs, so that no exit sits between a prefetch and
// its use for the compiler to sink the prefetch behind); each step is one multiply independent
// of the chain and one add on it. Reads stay inside the stage (positions < kA1ShortRow).
template <int HD>
__device__ __forceinline__ float a1_short_chain(const float* col, const float* pj, int n) {
    constexpr int C = 16, LIM = kA1ShortRow - C;
    float ea[C], va[C], eb[C], vb[C];
    auto ld = [&](float (&e)[C], float (&v)[C], int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < C; i += 4) {
            const float4 q = *reinterpret_cast<const float4*>(pj + j0 + i);
            e[i] = q.x, e[i + 1] = q.y, e[i + 2] = q.z, e[i + 3] = q.w;
        }
#pragma unroll
        for (int i = 0; i < C; i++) v[i] = col[(j0 + i) * HD];
    };
    float o = 0.f;
    auto add = [&](const float (&e)[C], const float (&v)[C]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < C; i++) o += e[i] * v[i];
    };
    // the partial last chunk: positions past the row add +0, which leaves o unchanged (o is
    // never -0: it starts at +0, and a sum that cancels rounds to +0)
    auto add_tail = [&](const float (&e)[C], const float (&v)[C], int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < C; i++) {
            const float t = e[i] * v[i];
            o += j0 + i < n ? t : 0.f;
        }
    };
    const int nfull = n / C;
    ld(ea, va, 0);
    int c = 0;
    // scheduling barriers keep each chunk's reads ahead of the previous chunk's adds
    for (; c + 2 <= nfull; c += 2) {  // no exit inside the body: the prefetches stay where written
        ld(eb, vb, (c + 1) * C);
        __builtin_amdgcn_sched_barrier(0);
        add(ea, va);
        __builtin_amdgcn_sched_barrier(0);
        ld(ea, va, min((c + 2) * C, LIM));
        __builtin_amdgcn_sched_barrier(0);
        add(eb, vb);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (c < nfull) {
        ld(eb, vb, min((c + 1) * C, LIM));
        __builtin_amdgcn_sched_barrier(0);
        add(ea, va);
        __builtin_amdgcn_sched_barrier(0);
        add_tail(eb, vb, (c + 1) * C);
    } else {
        add_tail(ea, va, c * C);
    }
    return o;
}

// One producer step: when the tile at t0 exists (a uniform branch), its V rows as fp32 (the edge
// form when it reaches the row's end) and its barrier; then, on every path, v refilled with the
// rows three tiles on. The loads are unconditional so that every path through a group of three
// steps leaves the same loads in flight, and the compiler's wait before a tile's stores leaves
// the later tiles' loads outstanding.
template <int HD>
__device__ __forceinline__ void a1_produce(uint2 (&v)[A1Split<HD>::IPT], float* buf, const uint16_t* vb,
                                           const uint16_t* V, int t0, int p, int pos, int n, int last) {
    if (t0 < n) {
        if (t0 + kA1Tile < n) a1_stage_tile<HD, false>(v, buf, vb, t0, p, pos, n);
        else a1_stage_tile<HD, true>(v, buf, vb, t0, p, pos, n);
    }
    a1_load_v<HD>(v, V, t0 + 3 * kA1Tile, p, last);
    if (t0 < n) hy_lds_barrier();
}

// The query head of this k_attn1 workgroup. Workgroups go to the 8 XCDs round-robin (workgroup b
// on XCD b % 8), each XCD with its own L2: consecutive heads share an XCD (heads 2x, 2x + 1 on XCD
// x for 16 heads), so a KV head's K and V rows are fetched by half as many L2s as in id order
// (measured 5.5x the algorithmic bytes in id order at 4 query heads per KV head). Head counts
// that are not a multiple of 8 keep id order.
__device__ __forceinline__ int a1_head(int heads) {
    const int b = blockIdx.x;
    return heads % 8 ? b : (b % 8) * (heads / 8) + b / 8;
}

// LDS of one head's attention.
template <int HD>
struct A1Smem {
    alignas(16) float ex[(kA1MaxCtx + kA1Tile - 1) / kA1Tile * kA1Tile];  // e_j = expf(s_j - max), then p_j
    union {
        HyExactLdsT<kA1Waves> exs;            // the softmax sum of long rows
        alignas(16) float prod[2][kA1Tile * HD];  // then the products of two tiles, [j][d]
    };
    alignas(16) float scr[2][HD];
    alignas(16) float qn[HD];
    alignas(16) uint16_t kb[HD];
    alignas(16) uint16_t vb[HD];
    float red[kA1Waves];
    float stat;
    uint64_t etab[32];  // expf table
};

// Phases 1-4 of one head's attention, every thread of the workgroup: this token's rows (x:
// q / k / v elements lane + 64 i for wavefronts 0 / 1 / 2), its RoPE row (rc, rs) and the q / k
// norm weights (nw) are loaded; the key rows of the first pass (kA, rows below pos) and, in the
// producer wavefronts (2-7), the first V tile (v0) are in flight.
template <int HD>
__device__ __forceinline__ void a1_core(const Attn1Args& a, A1Smem<HD>& S, const float (&x)[HD / 64],
                                        const float (&rc)[HD / 64], const float (&rs)[HD / 64],
                                        const float (&nw)[HD / 64], uint4 (&kA)[HD / 8], uint2 (&v0)[A1Split<HD>::IPT],
                                        uint2 (&v1)[A1Split<HD>::IPT], int pos, uint64_t etv) {
    constexpr int KV4 = HD / 8;                 // 16-byte pieces of one K / V row
    constexpr int RPL = HD / 64;                // row elements per lane
    constexpr int PASSES = kA1MaxCtx / kA1Threads;
    static_assert(kA1Waves == 8 && KV4 % 4 == 0, "8 wavefronts");
    float* ex = S.ex;
    float(&scr)[2][HD] = S.scr;
    float* qn = S.qn;
    uint16_t* kb = S.kb;
    uint16_t* vb = S.vb;
    float* red = S.red;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = a1_head(a.heads);
    const int group = a.heads / a.kv_heads;
    const int g = h / group;
    const int half = a.rope_half;
    const int cap = a.ctx - 1;
    const uint16_t* K = a.kc + (size_t)g * a.ctx * HD;
    const uint16_t* V = a.vc + (size_t)g * a.ctx * HD;
    const bool prd = wave >= 2;
    const int pp = prd ? tid - 128 : lane;  // producer index (other wavefronts: any valid one)
    const int n = pos + 1;
    uint4 kB[KV4];
    uint2 v2[A1Split<HD>::IPT];

    // 1. RoPE + RMSNorm of q (wavefront 0) and k (1), bf16 of k and v
    if (wave < 2) {
        float y[RPL];
        rope_norm_wave<HD>(x, scr[wave], rc, rs, half, nw, a.eps, lane, y);
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            if (wave == 0) qn[lane + 64 * i] = y[i];
            else kb[lane + 64 * i] = hy_to_bf16(y[i]);
        }
    } else if (wave == 2) {
#pragma unroll
        for (int i = 0; i < RPL; i++) vb[lane + 64 * i] = hy_to_bf16(x[i]);
    }
    // LDS only: a full __syncthreads would also wait for every key and V row in flight
    hy_lds_barrier();
    // the bf16 k, v of this position (src/model.c:842-847), stored once per KV head
    if (h % group == 0 && tid < HD) {
        const size_t off = ((size_t)g * a.ctx + pos) * HD + tid;
        a.kc[off] = kb[tid];
        a.vc[off] = vb[tid];
    }

    // 2. scores s_j = dot_bf16(q, K_j) * (1/sqrtf(hd)) for j = tid + 512 p, kept in registers;
    //    key `pos` is this token's kb; the next pass's rows load while this one is scored
    const float scale = 1.0f / sqrtf((float)HD);
    float sv[PASSES];
    float lmax = -__builtin_inff();
    const bool pair = n <= kA1PairRow;  // short rows: key tid / 2 on a pair of lanes (loaded at entry)
    if (pair) {
        const int m = tid >> 1;
        if (m < n) {
            if (m == pos) a1_load_key<HD>(kA, kb, 0);
            sv[0] = a1_score_pair<HD>(kA, qn, tid & 1, scale);
            lmax = sv[0];
        }
    }
#pragma unroll
    for (int p = 0; p < PASSES; p += 2) {
        if (pair) break;
        const int j0 = p * kA1Threads + tid, j1 = j0 + kA1Threads;
        if (j0 - tid >= n) break;
        if (j1 - tid < n) a1_load_key<HD>(kB, K, min(j1, cap));
        if (j0 < n) {
            if (j0 == pos) a1_load_key<HD>(kA, kb, 0);
            sv[p] = a1_score<HD>(kA, qn, scale);
            lmax = fmaxf(lmax, sv[p]);
        }
        if (j1 - tid >= n) break;
        if (j1 + kA1Threads - tid < n) a1_load_key<HD>(kA, K, min(j1 + kA1Threads, cap));
        if (j1 < n) {
            if (j1 == pos) a1_load_key<HD>(kB, kb, 0);
            sv[p + 1] = a1_score<HD>(kB, qn, scale);
            lmax = fmaxf(lmax, sv[p + 1]);
        }
    }
    // V tiles 1 and 2 of long rows (rows clamped below the position), by the producer
    // wavefronts only: both, so that the same loads follow tile 0's on every path and the
    // producers' waits leave them out (short rows loaded tile 1 at entry).
    const int last = max(pos - 1, 0);
    if (prd && n > kA1ShortRow) {
        a1_load_v<HD>(v1, V, kA1Tile, pp, last);
        a1_load_v<HD>(v2, V, 2 * kA1Tile, pp, last);
    }
    a1_fence();  // issued here, not next to their first use
    lmax = hy_wave_max(lmax);
    if (lane == 0) red[wave] = lmax;
    if (tid < 32) S.etab[tid] = etv;
    hy_lds_barrier();

    // 3. softmax (src/model.c:781-789): max (order-free), e_j = expf(s_j - max), their sum in
    //    position order, inv = 1 / sum. Short rows: the lane-serial chain of wavefront 0; long
    //    ones: the exact segmented form over 8 consecutive positions per thread.
    float inv;
    {
        float mx = red[0];
#pragma unroll
        for (int w = 1; w < kA1Waves; w++) mx = fmaxf(mx, red[w]);
#pragma unroll
        for (int p = 0; p < PASSES; p++) {
            const int j = p * kA1Threads + tid;
            if (pair) {
                // +0 past the row to the next multiple of 32: the lane-serial sum then reads whole
                // 32-value groups (adding +0 leaves a sum of non-negative terms unchanged)
                const int m = tid >> 1;
                if ((tid & 1) == 0 && m < (n + 31) / 32 * 32) ex[m] = m < n ? hy_expf_tab(sv[0] - mx, S.etab) : 0.f;
                break;
            }
            if (j - tid >= n) break;
            if (j < n) ex[j] = hy_expf_tab(sv[p] - mx, S.etab);
        }
        hy_lds_barrier();
        if (n <= kA1SerialSum) {
            if (wave == 0) {
                const float sum = hy_wave_seq_sum(ex, (n + 31) / 32 * 32, lane);  // the same value in every lane
                if (lane == 0) S.stat = 1.0f / sum;
                if (n <= kA1ShortRow) {  // short rows: p_j = e_j * (1 / sum) in place, once per position
                    const float iv = 1.0f / sum;
                    for (int j = lane; j < n; j += 64) ex[j] = ex[j] * iv;
                }
            } else if (n <= kA1ShortRow && prd) {  // meanwhile the producers stage V whole
                a1_stage_v<HD>(v0, &S.prod[0][0], vb, 0, pp, pos, n);
                if (n > kA1Tile) a1_stage_v<HD>(v1, &S.prod[0][0], vb, kA1Tile, pp, pos, n);
            }
            hy_lds_barrier();
            inv = S.stat;
        } else {
            const int e0 = 8 * tid;
            float e[8];
#pragma unroll
            for (int i = 0; i < 8; i++) e[i] = 0.f;
            if (e0 < n) {
                const float4 s0 = *reinterpret_cast<const float4*>(ex + e0);
                const float4 s1 = *reinterpret_cast<const float4*>(ex + e0 + 4);
                const float ev[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
                for (int i = 0; i < 8; i++) e[i] = e0 + i < n ? ev[i] : 0.f;
            }
            inv = 1.0f / hy_block_exact_sum8<kA1Waves, false>(e, S.exs, wave, lane);
        }
        if (n > kA1ShortRow) {
            // p_j = e_j * (1 / sum), once per position; +0 past the row to the end of its last tile
            const int end = (n + kA1Tile - 1) / kA1Tile * kA1Tile;
            for (int j = tid; j < end; j += kA1Threads) ex[j] = j < n ? ex[j] * inv : 0.f;
            hy_lds_barrier();  // and the tiles reuse the sum's LDS
        }
    }

    // 4. o[d] = sum_j p_j * V_j[d] in position order (axpy_bf16). Barrier t: tile t is in
    //    buffer t % 2, and tile t - 1's buffer has been read. Wavefronts 0 .. HD/64 - 1 walk tile
    //    t after barrier t; the producers convert tile t's V rows before it, with V three tiles
    //    ahead, in groups of three steps (one loop exit; steps past the row only load).
    // Short rows: every lane of wavefronts 0 .. HD/64 - 1 walks its dimension over the staged V.
    if (n <= kA1ShortRow) {
        static_assert(kA1ShortRow <= kA1SerialSum && kA1ShortRow * HD <= 2 * kA1Tile * HD, "staged V fits");
        if (wave < HD / 64) a.ao[(size_t)h * HD + tid] = a1_short_chain<HD>(&S.prod[0][0] + tid, ex, n);
        return;
    }
    const int tiles = (n + kA1Tile - 1) / kA1Tile;
    if (wave < HD / 64) {
        __builtin_amdgcn_s_setprio(3);  // the chain is the critical path: its adds issue first
        float o = 0.f;
        for (int t = 0; t < tiles; t++) {
            hy_lds_barrier();
            const int cnt = min(kA1Tile, n - t * kA1Tile);
            a1_chain<HD>(S.prod[t & 1] + tid, ex + t * kA1Tile, (cnt + kA1Chunk - 1) / kA1Chunk, o);
        }
        a.ao[(size_t)h * HD + tid] = o;
    } else if (prd) {
        for (int t = 0; t < tiles; t += 3) {
            const int t0 = t * kA1Tile;
            a1_produce<HD>(v0, S.prod[t & 1], vb, V, t0, pp, pos, n, last);
            a1_produce<HD>(v1, S.prod[(t + 1) & 1], vb, V, t0 + kA1Tile, pp, pos, n, last);
            a1_produce<HD>(v2, S.prod[t & 1], vb, V, t0 + 2 * kA1Tile, pp, pos, n, last);
        }
    } else {
        for (int t = 0; t < tiles; t++) hy_lds_barrier();
    }
}

template <int HD>
__global__ __launch_bounds__(kA1Threads) void k_attn1(Attn1Args a) {
    constexpr int RPL = HD / 64;
    __shared__ A1Smem<HD> S;
    // Every kernel argument in one round of scalar loads, pinned in SGPRs before use: the
    // per-wavefront selections below would otherwise chain dependent loads of the arguments.
    hy_sgpr_pin(a.q), hy_sgpr_pin(a.k), hy_sgpr_pin(a.v), hy_sgpr_pin(a.kc), hy_sgpr_pin(a.vc),
        hy_sgpr_pin(a.q_norm), hy_sgpr_pin(a.k_norm), hy_sgpr_pin(a.rope_cos), hy_sgpr_pin(a.rope_sin),
        hy_sgpr_pin(a.pos_dev), hy_sgpr_pin(a.rope_cur), hy_sgpr_pin(a.pos0), hy_sgpr_pin(a.ao), hy_sgpr_pin(a.heads),
        hy_sgpr_pin(a.kv_heads), hy_sgpr_pin(a.rope_half), hy_sgpr_pin(a.ctx), hy_sgpr_pin(a.eps);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = a1_head(a.heads);
    const int g = h / (a.heads / a.kv_heads);
    const int half = a.rope_half;
    const uint16_t* K = a.kc + (size_t)g * a.ctx * HD;
    const uint16_t* V = a.vc + (size_t)g * a.ctx * HD;
    const bool prd = wave >= 2;
    const int pp = prd ? tid - 128 : lane;

    // 0. loads: this token's q / k / v row for wavefronts 0 / 1 / 2 with the norm weights, the
    //    position (scalar) and its RoPE row (rope_cur when the position lives in device memory),
    //    then the key rows of the first pass (those below the position) and the first V tile
    // The rows and norm weights first: loads return in issue order.
    float x[RPL], rc[RPL], rs[RPL], nw[RPL];
    const uint64_t etv = tid < 32 ? hy_exp_tab_entry(tid) : 0;  // expf table entry, into LDS before the max
    {
        const float* src = wave == 0 ? a.q + (size_t)h * HD : (wave == 1 ? a.k + (size_t)g * HD : a.v + (size_t)g * HD);
        const float* nsrc = wave == 0 ? a.q_norm : a.k_norm;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int d = lane + 64 * i;
            x[i] = src[d];
            nw[i] = nsrc[d];
        }
    }
    // The position by a scalar load waited for on its own: read as *pos_dev it compiled to a
    // vector load whose wait covered the row loads just issued (the previous kernel's output,
    // about 1.8 us), and the key and V loads that need the position went out only after them.
    // (Issuing the pair form's key rows and the V tiles before the position, clamped, was slower:
    // their 64 KB delayed the rows the RoPE needs first, 1022 -> 993 tok/s.)
    __builtin_amdgcn_sched_barrier(0);
    const int pos = a.pos_dev ? hy_sload_i32(a.pos_dev) : a.pos0;
    {
        const float* cs = a.rope_cur ? a.rope_cur : a.rope_cos + (size_t)pos * half;
        const float* sn = a.rope_cur ? a.rope_cur + half : a.rope_sin + (size_t)pos * half;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int d = lane + 64 * i, t = d < half ? d : (d < 2 * half ? d - half : 0);
            rc[i] = cs[t];
            rs[i] = sn[t];
        }
    }
    a1_fence();  // the row loads go out first: loads return in issue order
    uint4 kA[HD / 8];
    if (pos < kA1PairRow) {  // the score phase's pair form: key tid / 2
        if ((tid >> 1) < pos) a1_load_key<HD>(kA, K, tid >> 1);
    } else if (tid < pos) {
        a1_load_key<HD>(kA, K, tid);
    }
    uint2 v0[A1Split<HD>::IPT], v1[A1Split<HD>::IPT];
    a1_load_v<HD>(v0, V, 0, pp, max(pos - 1, 0));
    // short rows past one tile: the producers' second tile too, staged during the softmax sum
    if (prd && pos >= kA1Tile && pos < kA1ShortRow) a1_load_v<HD>(v1, V, kA1Tile, pp, pos - 1);
    a1_fence();
    a1_core<HD>(a, S, x, rc, rs, nw, kA, v0, v1, pos, etv);
}

hipError_t launch_attn1(const Attn1Args& a, hipStream_t s) {
    if (a.heads % a.kv_heads || 2 * a.rope_half > a.hdim || a.ctx > kA1MaxCtx) return hipErrorNotSupported;
    switch (a.hdim) {
    case 64: k_attn1<64><<<a.heads, kA1Threads, 0, s>>>(a); break;
    case 128: k_attn1<128><<<a.heads, kA1Threads, 0, s>>>(a); break;
    default: return hipErrorNotSupported;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ split form for long rows
//
// The same attention as k_attn1 in two kernels, so that long rows use many CUs:
//   k_attn_scores, one 512-thread workgroup per (KV head, segment of kSplitSeg positions):
//     RoPE + RMSNorm of the group's q heads (recomputed by every workgroup) and, in the workgroup
//     whose segment holds the position, of this token's k, with the bf16 KV store at the
//     position; then wavefront w scores q head w % 4 over half of the segment, one key per pair
//     of lanes in dot_bf16's order; the scores and each half-segment's maximum go to global
//     memory.
//   k_attn_out, one 512-thread workgroup per (query head, kSoDims output dimensions): the maximum
//     of the segment maxima (order-free), e_j = expf(s_j - max) (positions dealt to the threads
//     round-robin, through LDS), their sum in position order by the 8-wavefront exact segmented
//     sum (rows longer than kSplitWin in chunks, each later chunk taking the running sum as its
//     first addend, which continues the same sequential sum), p_j = e_j * (1 / sum), then
//     o[d] += p_j * V_j[d] in position order: wavefronts 1-3 and 5-7 form the products
//     p_j * V_j[d] (rounded to fp32, as the reference's multiply) into [d][j] tiles of 256
//     positions, and wavefront 0 (one lane per dimension) adds them in position order, four per
//     LDS read, with only the dependent adds on its critical path. Wavefront 4, which shares
//     wavefront 0's SIMD, only keeps the barriers: an instruction it issued would delay the
//     chain's next add (measured 8.9 against 6.4 cycles an add). The output chains of a head are sequential
//     in position, so the work spreads over the dimensions: 16 a workgroup keeps the products
//     of a tile (4096) off the chain's path and puts 8 workgroups on each head.

namespace {

constexpr int kSpThreads = 512;                // k_attn_scores: eight wavefronts
constexpr int kSpGridX = 128;                  // score workgroups per KV head (more segments loop)
constexpr int kSoThreads = 512;                // k_attn_out
constexpr int kSoNW = kSoThreads / 64;         // its wavefronts
constexpr int kSoDims = 16;                    // output dimensions per k_attn_out workgroup
constexpr int kSoDG = kSoDims / 8;             // 16-byte V pieces (8 dimensions) per position
constexpr int kSoTile = 256;                   // positions per product tile
constexpr int kSoPad = kSoTile + 4;            // [d][j] row length (16-byte rows)
constexpr int kSoPieces = kSoTile * kSoDG;     // (position, 8 dimensions) pieces of a tile
constexpr int kSoProd = kSoThreads - 128;      // producer threads (wavefronts 1-3 and 5-7)
constexpr int kSoPPT = (kSoPieces + kSoProd - 1) / kSoProd;  // pieces per producer thread
constexpr int kSoEPT = kSplitWin / kSoThreads;               // positions of a window per thread
static_assert(kSoEPT == 8, "hy_block_exact_sum8 takes eight addends a thread");
static_assert(kSplitWin % kSoTile == 0, "windows of whole tiles");
static_assert(kSoTile % 32 == 0 && kSoDims % 8 == 0 && kSoDims <= 64, "swizzle within 32 positions; whole pieces");

struct SoSmem {
    alignas(16) float pj[kSplitWin];  // e_j, then p_j, of the current window
    union {
        HyExactLdsT<kSoNW> exs;                       // the softmax sum
        alignas(16) float prod[2][kSoDims][kSoPad];   // then two product tiles [d][j]
    };
    float red[kSoNW];
    uint64_t etab[32];  // expf table
};

}  // namespace

template <int HD>
__global__ __launch_bounds__(kSpThreads) void k_attn_scores(Attn1Args a) {
    constexpr int RPL = HD / 64;
    constexpr int HW = kSpThreads / 128;               // wavefronts per half of the workgroup (head slots)
    constexpr int QPW = kSplitMaxGroup / HW;           // query heads per wavefront at most
    constexpr int NW = kSpThreads / 64;
    __shared__ alignas(16) float qn[NW][QPW][HD];      // each wavefront's own normalized q rows
    __shared__ alignas(16) float scr[NW][HD];
    __shared__ alignas(16) uint16_t kb[NW][HD];        // this token's bf16 k, in each wavefront that scores it
    hy_sgpr_pin(a.q), hy_sgpr_pin(a.k), hy_sgpr_pin(a.v), hy_sgpr_pin(a.kc), hy_sgpr_pin(a.vc),
        hy_sgpr_pin(a.q_norm), hy_sgpr_pin(a.k_norm), hy_sgpr_pin(a.rope_cos), hy_sgpr_pin(a.rope_sin),
        hy_sgpr_pin(a.pos_dev), hy_sgpr_pin(a.rope_cur), hy_sgpr_pin(a.pos0), hy_sgpr_pin(a.heads),
        hy_sgpr_pin(a.kv_heads), hy_sgpr_pin(a.rope_half), hy_sgpr_pin(a.ctx), hy_sgpr_pin(a.eps), hy_sgpr_pin(a.sc),
        hy_sgpr_pin(a.segmax), hy_sgpr_pin(a.sc_stride), hy_sgpr_pin(a.seg_stride);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = blockIdx.y, group = a.heads / a.kv_heads;
    const int half = a.rope_half;
    const uint16_t* K = a.kc + (size_t)g * a.ctx * HD;
    // wavefront w scores the group's q heads w % HW, w % HW + HW, ... for the half w / HW of the
    // segment's positions, one key per pair of lanes. Nothing is shared between wavefronts:
    // each RoPEs and norms its own q heads (the two halves' wavefronts of a head both do), and
    // the wavefronts whose keys include the position RoPE and norm this token's k themselves,
    // so the workgroup has no barrier (one cost 0.7 us waiting for the slowest row's arrival).
    const int slot = wave % HW, sh = wave / HW;
    const bool hasq = slot < group;
    const int par = lane & 1;

    // 0. q row and norm weights, this token's k and v rows, the first segment's key rows (clamped
    //    inside the cache: which of them lie below the position is known only after its read,
    //    and the rows arrive about 2.5 us after issue), then the position (scalar) and its RoPE row
    float x[RPL], nw[RPL], kx[RPL], knw[RPL], vx[RPL];
#pragma unroll
    for (int i = 0; i < RPL; i++) {
        const int d = lane + 64 * i;
        if (hasq) x[i] = a.q[(size_t)(g * group + slot) * HD + d], nw[i] = a.q_norm[d];
        kx[i] = a.k[(size_t)g * HD + d], knw[i] = a.k_norm[d], vx[i] = a.v[(size_t)g * HD + d];
    }
    const int koff = sh * (kSplitSeg / 2) + (lane >> 1);  // this lane's key within a segment
    uint4 kr[HD / 8];
    if (hasq) a1_load_key<HD>(kr, K, min((int)blockIdx.x * kSplitSeg + koff, a.ctx - 1));
    __builtin_amdgcn_sched_barrier(0);
    const int pos = a.pos_dev ? hy_sload_i32(a.pos_dev) : a.pos0;
    const int n = pos + 1, nseg = (n + kSplitSeg - 1) / kSplitSeg;
    if ((int)blockIdx.x >= nseg || !hasq) return;  // uniform: no work for this workgroup / wavefront
    // this wavefront scores the position's key: its workgroup has the last segment and its half
    // of the segment holds the position
    const bool kw = (nseg - 1) % (int)gridDim.x == (int)blockIdx.x && sh == (pos % kSplitSeg) / (kSplitSeg / 2);
    float rc[RPL], rs[RPL];
    {
        const float* cs = a.rope_cur ? a.rope_cur : a.rope_cos + (size_t)pos * half;
        const float* sn = a.rope_cur ? a.rope_cur + half : a.rope_sin + (size_t)pos * half;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int d = lane + 64 * i, t = d < half ? d : (d < 2 * half ? d - half : 0);
            rc[i] = cs[t];
            rs[i] = sn[t];
        }
    }
    a1_fence();

    // 1. RoPE + RMSNorm (src/model.c:836-841) of the wavefront's q heads and, where it scores the
    //    position, of this token's k (bf16; stored at the position with its v by the head slot 0
    //    wavefront, src/model.c:842-847)
    if (kw) {
        float y[RPL];
        rope_norm_wave<HD>(kx, scr[wave], rc, rs, half, knw, a.eps, lane, y);
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int d = lane + 64 * i;
            const uint16_t kq = hy_to_bf16(y[i]);
            kb[wave][d] = kq;
            if (slot == 0) {
                const size_t off = ((size_t)g * a.ctx + pos) * HD + d;
                a.kc[off] = kq;
                a.vc[off] = hy_to_bf16(vx[i]);
            }
        }
    }
    for (int hq = slot, k = 0; hq < group; hq += HW, k++) {
        if (hq != slot) {
#pragma unroll
            for (int i = 0; i < RPL; i++) x[i] = a.q[(size_t)(g * group + hq) * HD + lane + 64 * i];
        }
        float y[RPL];
        rope_norm_wave<HD>(x, scr[wave], rc, rs, half, nw, a.eps, lane, y);
#pragma unroll
        for (int i = 0; i < RPL; i++) qn[wave][k][lane + 64 * i] = y[i];
    }
    // the wavefront reads its own LDS rows from here on
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // 2. scores s_j = dot_bf16(q, K_j) * (1/sqrtf(hd)) (src/model.c:778-782) of this workgroup's
    //    segments, key pos from this token's bf16 k; the maximum of each kSplitMaxSeg positions
    //    (order-free)
    const float scale = 1.0f / sqrtf((float)HD);
    for (int sgm = blockIdx.x; sgm < nseg; sgm += gridDim.x) {
        const int r = sgm * kSplitSeg + koff;
        if (sgm != (int)blockIdx.x && r < pos) a1_load_key<HD>(kr, K, r);
        if (r == pos) a1_load_key<HD>(kr, kb[wave], 0);
        for (int hq = slot, k = 0; hq < group; hq += HW, k++) {
            const float s = a1_score_pair<HD>(kr, qn[wave][k], par, scale);
            const int hh = g * group + hq;
            if (r < n && par == 0) a.sc[(size_t)hh * a.sc_stride + r] = s;
            const float m = hy_wave_max(r < n ? s : -__builtin_inff());
            if (lane == 0) a.segmax[(size_t)hh * a.seg_stride + sgm * 2 + sh] = m;
        }
    }
}

namespace {

// Product tile layout: buf[d][c], d the dimension (of this workgroup's kSoDims), c a swizzled
// position: position j of the tile sits at column j ^ (4 * (d / 8)). The XOR moves whole groups
// of four positions within aligned groups of 32, so the chain's 16-byte reads of four
// consecutive positions stay contiguous, and the producers' stores of one instruction (32
// positions times two 8-dimension groups) spread over the LDS banks.

// V pieces of the tile at t0 for producer thread pt: piece q = pt + kSoProd k is position
// t0 + q / kSoDG, dimensions 8 (q % kSoDG) .. + 8 of this workgroup's kSoDims (V is offset to
// them); rows clamped inside the cache (pieces past the row are never added). Every load is
// issued, also for pieces past the tile's (q clamped, the value unused): with a conditional load
// the compiler cannot count the loads in flight and waits for all of them.
template <int HD>
__device__ __forceinline__ void so_load_v(uint4 (&v)[kSoPPT], const uint16_t* V, int t0, int pt, int cap) {
#pragma unroll
    for (int k = 0; k < kSoPPT; k++) {
        const int q = min(pt + kSoProd * k, kSoPieces - 1);
        v[k] = *reinterpret_cast<const uint4*>(V + (size_t)min(t0 + q / kSoDG, cap) * HD + 8 * (q % kSoDG));
    }
}

// The products p_j * V_j[d] of a tile (rounded to fp32, axpy_bf16's multiply) into buf.
__device__ __forceinline__ void so_products(const uint4 (&v)[kSoPPT], float (*buf)[kSoPad], const float* pj, int pt) {
#pragma unroll
    for (int k = 0; k < kSoPPT; k++) {
        const int q = pt + kSoProd * k;
        if (q < kSoPieces) {
            const int j = q / kSoDG, dg = q % kSoDG;
            const float p = pj[j];
            float f[8];
            bf16x8f(v[k], f);
            const int c = j ^ (4 * dg);  // the column of position j in rows 8 dg .. 8 dg + 7
#pragma unroll
            for (int i = 0; i < 8; i++) buf[8 * dg + i][c] = p * f[i];
        }
    }
}

// o += the products of positions 0 .. cnt - 1 of lane d's row, one add at a time in position
// order (cnt uniform). Whole 32-position chunks run double-buffered: the reads of chunk c + 1 are
// issued before the 32 adds of chunk c, so an LDS round trip (longer than 16 dependent adds) is
// hidden; scheduling barriers keep the reads there. A partial last chunk adds +0 past cnt, which
// leaves o unchanged (o is never -0: it starts at +0, and a sum of nonzero addends that cancels
// rounds to +0).
__device__ __forceinline__ void so_chain(const float* row, int d, int cnt, float& o) {
    constexpr int CH = 32;  // positions per chunk
    const int sw = 4 * (d >> 3);
    auto ld = [&](float4 (&x)[CH / 4], int c) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < CH / 4; k++) x[k] = *reinterpret_cast<const float4*>(row + ((CH * c + 4 * k) ^ sw));
    };
    // 16 dependent adds as one block: one wait for all of its operands before it, and the
    // running sum kept in one register (the compiler otherwise waits on the LDS counter every
    // four to eight adds and moves the sum between registers: 8.7 against 6.4 cycles an add)
    auto add16 = [&](const float4& a, const float4& b, const float4& c, const float4& e) __attribute__((always_inline)) {
        asm volatile(
            "v_add_f32 %0, %0, %1\n\tv_add_f32 %0, %0, %2\n\tv_add_f32 %0, %0, %3\n\tv_add_f32 %0, %0, %4\n\t"
            "v_add_f32 %0, %0, %5\n\tv_add_f32 %0, %0, %6\n\tv_add_f32 %0, %0, %7\n\tv_add_f32 %0, %0, %8\n\t"
            "v_add_f32 %0, %0, %9\n\tv_add_f32 %0, %0, %10\n\tv_add_f32 %0, %0, %11\n\tv_add_f32 %0, %0, %12\n\t"
            "v_add_f32 %0, %0, %13\n\tv_add_f32 %0, %0, %14\n\tv_add_f32 %0, %0, %15\n\tv_add_f32 %0, %0, %16"
            : "+v"(o)
            : "v"(a.x), "v"(a.y), "v"(a.z), "v"(a.w), "v"(b.x), "v"(b.y), "v"(b.z), "v"(b.w), "v"(c.x), "v"(c.y),
              "v"(c.z), "v"(c.w), "v"(e.x), "v"(e.y), "v"(e.z), "v"(e.w));
    };
    auto add = [&](const float4 (&x)[CH / 4]) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < CH / 4; k += 4) add16(x[k], x[k + 1], x[k + 2], x[k + 3]);
    };
    constexpr int C = kSoTile / CH;
    const int full = cnt / CH;
    float4 A[CH / 4], B[CH / 4];
    ld(A, 0);
    int c = 0;
    for (; c + 2 <= full; c += 2) {  // A holds chunk c
        ld(B, c + 1);
        __builtin_amdgcn_sched_barrier(0);
        add(A);
        __builtin_amdgcn_sched_barrier(0);
        ld(A, min(c + 2, C - 1));
        __builtin_amdgcn_sched_barrier(0);
        add(B);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (c < full) {  // an odd whole chunk
        add(A);
        c++;
        if (CH * c < cnt) ld(A, c);
    }
    if (CH * c < cnt) {
#pragma unroll
        for (int k = 0; k < CH / 4; k++) {
            const int j = CH * c + 4 * k;
            o += j < cnt ? A[k].x : 0.f;
            o += j + 1 < cnt ? A[k].y : 0.f;
            o += j + 2 < cnt ? A[k].z : 0.f;
            o += j + 3 < cnt ? A[k].w : 0.f;
        }
    }
}

}  // namespace

// The (query head, dimension part) of this k_attn_out workgroup. Workgroups go to the 8 XCDs
// round-robin (workgroup b on XCD b % 8), each XCD with its own L2: the ids are dealt so that the
// workgroups reading the same V lines (a KV head's 64 dimensions of every row, 128 bytes: the
// group's query heads times the four 16-dimension parts of the line) run on one XCD, which then
// fetches those lines once (dealt in id order, the eight parts of a head on eight XCDs fetched
// 4.9x the V and score bytes). Launches whose workgroup count is not a multiple of 8 keep id
// order.
template <int HD>
__device__ __forceinline__ void so_assign(int heads, int group, int& h, int& part) {
    constexpr int PARTS = HD / kSoDims, LPARTS = 64 / kSoDims, LINES = HD / 64;
    const int b = blockIdx.x, total = heads * PARTS;
    const int q = total % 8 ? b : (b % 8) * (total / 8) + b / 8;
    const int gs = group * LPARTS;  // workgroups of one (KV head, line)
    const int grp = q / gs, mem = q % gs;
    h = (grp / LINES) * group + mem / LPARTS;
    part = (grp % LINES) * LPARTS + mem % LPARTS;
}

template <int HD>
__global__ __launch_bounds__(kSoThreads) void k_attn_out(Attn1Args a) {
    constexpr int PARTS = HD / kSoDims;
    __shared__ SoSmem S;
    hy_sgpr_pin(a.vc), hy_sgpr_pin(a.pos_dev), hy_sgpr_pin(a.pos0), hy_sgpr_pin(a.ao), hy_sgpr_pin(a.heads),
        hy_sgpr_pin(a.kv_heads), hy_sgpr_pin(a.ctx), hy_sgpr_pin(a.sc), hy_sgpr_pin(a.segmax),
        hy_sgpr_pin(a.sc_stride), hy_sgpr_pin(a.seg_stride);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int h, part;
    so_assign<HD>(a.heads, a.heads / a.kv_heads, h, part);
    const int g = h / (a.heads / a.kv_heads);
    const uint16_t* V = a.vc + (size_t)g * a.ctx * HD + kSoDims * part;
    const bool prd = wave >= 1 && wave != 4;        // producer wavefronts
    const int pt = tid - (wave < 4 ? 64 : 128);     // producer index
    const int cap = a.ctx - 1;
    const float* sc = a.sc + (size_t)h * a.sc_stride;

    // 0. loads that do not wait for the position, oldest first (their waits then leave the
    //    younger ones in flight): this thread's scores of the first window (positions
    //    tid + kSoThreads i) and one segment maximum (masked by the position below), then the
    //    producers' V pieces of the first three tiles
    const uint64_t etv = tid < 32 ? hy_exp_tab_entry(tid) : 0;  // expf table entry, into LDS before the max
    float sv[kSoEPT];
#pragma unroll
    for (int i = 0; i < kSoEPT; i++) {
        const int j = tid + kSoThreads * i;
        sv[i] = j < a.sc_stride ? sc[j] : 0.f;
    }
    const float m0 = tid < a.seg_stride ? a.segmax[(size_t)h * a.seg_stride + tid] : -__builtin_inff();
    uint4 va[kSoPPT], vb[kSoPPT], vc[kSoPPT];
    if (prd) {
        so_load_v<HD>(va, V, 0, pt, cap);
        so_load_v<HD>(vb, V, kSoTile, pt, cap);
        so_load_v<HD>(vc, V, 2 * kSoTile, pt, cap);
    }
    a1_fence();
    const int pos = a.pos_dev ? hy_sload_i32(a.pos_dev) : a.pos0;  // not waiting for the V loads
    const int n = pos + 1, nseg = (n + kSplitMaxSeg - 1) / kSplitMaxSeg;  // segment maxima in use

    // 1. max over the segment maxima (src/model.c:781-782; order-free)
    float m = tid < nseg ? m0 : -__builtin_inff();
    for (int i = tid + kSoThreads; i < nseg; i += kSoThreads) m = fmaxf(m, a.segmax[(size_t)h * a.seg_stride + i]);
    m = hy_wave_max(m);
    if (lane == 0) S.red[wave] = m;
    if (tid < 32) S.etab[tid] = etv;
    hy_lds_barrier();
    float mx = S.red[0];
#pragma unroll
    for (int w = 1; w < kSoNW; w++) mx = fmaxf(mx, S.red[w]);

    // 2. e_j = expf(s_j - max) and their sum in position order (src/model.c:784-785); the sum
    //    takes thread t's addends as positions 8t .. 8t + 7 of a chunk
    const bool one = n <= kSplitWin;
    float sum;
    if (one) {
        // each thread forms the exponentials of its round-robin positions (at most
        // ceil(n / kSoThreads) each), then reads its eight consecutive ones back
#pragma unroll
        for (int i = 0; i < kSoEPT; i++) {
            const int j = tid + kSoThreads * i;
            if (j < n) S.pj[j] = hy_expf_tab(sv[i] - mx, S.etab);
        }
        hy_lds_barrier();
        float e[8];
        const int e0 = 8 * tid;
        if (e0 < n) {
            const float4 x0 = *reinterpret_cast<const float4*>(S.pj + e0);
            const float4 x1 = *reinterpret_cast<const float4*>(S.pj + e0 + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int i = 0; i < 8; i++) e[i] = e0 + i < n ? xv[i] : 0.f;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) e[i] = 0.f;
        }
        sum = hy_block_exact_sum8<kSoNW, false>(e, S.exs, wave, lane);
        // p_j = e_j * inv over this thread's own eight positions (read back above, so no other
        // thread writes them); the first tile's barrier publishes them
        const float inv = 1.0f / sum;
        if (e0 < n) {
            float p[8];
#pragma unroll
            for (int i = 0; i < 8; i++) p[i] = e[i] * inv;
            *reinterpret_cast<float4*>(S.pj + e0) = make_float4(p[0], p[1], p[2], p[3]);
            *reinterpret_cast<float4*>(S.pj + e0 + 4) = make_float4(p[4], p[5], p[6], p[7]);
        }
    } else {
        // chunks of kSplitWin addends; a later chunk's first addend is the running sum, so the
        // chunk continues the one sequential sum. The score row is only read: the head's other
        // workgroups read the same row, so e_j is formed again from s_j where the windows of p_j
        // are filled below.
        float e[8];
        float carry = 0.f;
        for (int base = 0, c = 0; base < n; c++) {
            const int off = c ? 1 : 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int idx = 8 * tid + i, j = base + idx - off;
                if (off && idx == 0) {
                    e[i] = carry;
                } else if (j < n) {
                    e[i] = hy_expf_tab(sc[j] - mx, S.etab);
                } else {
                    e[i] = 0.f;
                }
            }
            carry = hy_block_exact_sum8<kSoNW, false>(e, S.exs, wave, lane);
            __syncthreads();  // the sum's LDS is written again by the next chunk
            base += kSplitWin - off;
        }
        sum = carry;
    }
    const float inv = 1.0f / sum;

    // 3. o[d] = sum_j p_j * V_j[d] in position order (axpy_bf16), p_j = e_j * inv. Rows past
    //    kSplitWin: the producers fill p_j into LDS a window at a time (a barrier after each
    //    fill). Then one barrier per tile: before barrier t the producers have formed tile t into
    //    buffer t % 2, after it the chain adds tile t (tile t - 1's buffer was read before
    //    barrier t, when the producers fill it with tile t + 1).
    constexpr int WT = kSplitWin / kSoTile;  // tiles per window
    const int tiles = (n + kSoTile - 1) / kSoTile;
    if (wave == 4) {
        // the chain's SIMD neighbour: the barriers of the producers' steps and nothing else
        for (int t = 0; t < tiles; t++) {
            if (t % WT == 0) hy_lds_barrier();
            hy_lds_barrier();
        }
    } else if (!prd) {
        __builtin_amdgcn_s_setprio(3);  // the chain is the critical path: its adds issue first
        const int d = lane % kSoDims;   // lanes past kSoDims repeat a chain and store nothing
        const float* row = &S.prod[0][d][0];
        float o = 0.f;
        for (int t = 0; t < tiles; t++) {
            if (t % WT == 0) hy_lds_barrier();  // the window's p_j
            hy_lds_barrier();
            so_chain(row + (t & 1) * kSoDims * kSoPad, d, min(kSoTile, n - t * kSoTile), o);
        }
        if (lane < kSoDims) a.ao[(size_t)h * HD + kSoDims * part + lane] = o;
    } else {
        // one step per tile, unrolled by three over three register sets of V pieces, each
        // refilled three tiles ahead: every load is issued a full three tiles before its use and
        // no register copy waits on a recent load. Loads past the row read clamped rows.
        auto step = [&](uint4 (&v)[kSoPPT], int t) __attribute__((always_inline)) {
            if (t < tiles) {
                if (t % WT == 0) {
                    if (!one) {
                        const int w0 = t * kSoTile, wn = min(kSplitWin, n - w0);
                        for (int j = pt; j < wn; j += kSoProd) S.pj[j] = hy_expf_tab(sc[w0 + j] - mx, S.etab) * inv;
                    }
                    hy_lds_barrier();
                }
                so_products(v, S.prod[t & 1], S.pj + (t % WT) * kSoTile, pt);
                hy_lds_barrier();
            }
            so_load_v<HD>(v, V, (t + 3) * kSoTile, pt, cap);
        };
        for (int t = 0; t < tiles; t += 3) {
            step(va, t);
            step(vb, t + 1);
            step(vc, t + 2);
        }
    }
}

hipError_t launch_attn_split(const Attn1Args& a, hipStream_t s) {
    if (a.heads % a.kv_heads || a.heads / a.kv_heads > kSplitMaxGroup || 2 * a.rope_half > a.hdim || !a.sc ||
        !a.segmax || a.sc_stride < split_sc_stride(a.ctx) || a.seg_stride < split_seg_stride(a.ctx))
        return hipErrorNotSupported;
    const dim3 g1(min(split_seg_stride(a.ctx), kSpGridX), a.kv_heads);
    const int g2 = a.heads * (a.hdim / kSoDims);
    switch (a.hdim) {
    case 64:
        k_attn_scores<64><<<g1, kSpThreads, 0, s>>>(a);
        k_attn_out<64><<<g2, kSoThreads, 0, s>>>(a);
        break;
    case 128:
        k_attn_scores<128><<<g1, kSpThreads, 0, s>>>(a);
        k_attn_out<128><<<g2, kSoThreads, 0, s>>>(a);
        break;
    case 256:
        k_attn_scores<256><<<g1, kSpThreads, 0, s>>>(a);
        k_attn_out<256><<<g2, kSoThreads, 0, s>>>(a);
        break;
    default: return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace hy
