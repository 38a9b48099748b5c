// gfx950 kernels of the Hy-MT2 token loop. Every kernel reproduces the reference's scalar CPU
// arithmetic (src/kernels.c, src/model.c; HYMT2_ISA=scalar) bit for bit: integer block dots
// are exact in any order, and every fp32 reduction runs sequentially in the reference's order
// in one lane, while the parallel work (loads, int8 dot products, exponentials, elementwise
// ops) is spread over the wavefronts.
#include "hy_kernels.h"
#include "hy_mv_parts.h"

namespace hy {

// =========================================================================== Q8_K quantize

// One wavefront quantizes one 256-element block (src/kernels.c:128-165). Lane l owns elements
// 4l..4l+3. src and dst are flat pointers (LDS or global).
__device__ void q8k_quantize_wave(const float* src, HyQ8K* dst, int lane) {
    const float4 v4 = reinterpret_cast<const float4*>(src)[lane];
    const float e[4] = {v4.x, v4.y, v4.z, v4.w};
    uint32_t amax = 0;
    for (int i = 0; i < 4; i++) amax = max(amax, hy_fbits(e[i]) & 0x7fffffffu);
    amax = hy_wave_max_u(amax);
    uint32_t* dw = reinterpret_cast<uint32_t*>(dst);
    if (amax == 0) {  // all-zero block -> all-zero record
        for (int i = lane; i < 576 / 4; i += 64) dw[i] = 0;
        return;
    }
    int first = 256;
    for (int i = 3; i >= 0; i--)
        if ((hy_fbits(e[i]) & 0x7fffffffu) == amax) first = 4 * lane + i;
    first = hy_wave_min_i(first);
    const float vmax = src[first];
    const float iscale = -127.f / vmax;
    int q[4];
    for (int i = 0; i < 4; i++) {
        int r = (int)__builtin_rintf(iscale * e[i]);
        q[i] = r > 127 ? 127 : (r < -127 ? -127 : r);
    }
    const int s4 = q[0] + q[1] + q[2] + q[3];
    const int s16 = hy_quad_sum(s4);
    const int total = hy_wave_sum_i(s4);
    const uint32_t packed = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                            ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
    // natural order qs
    dw[320 / 4 + lane] = packed;
    // reordered copy: element c*64 + l*16 + i lands at qp[l*64 + {0,2,1,3}[c]*16 + i]
    const int c = lane >> 4, l = (lane >> 2) & 3, i0 = 4 * (lane & 3);
    const int seg = (c == 1) ? 2 : (c == 2 ? 1 : c);
    dw[(l * 64 + seg * 16 + i0) / 4] = packed;
    if ((lane & 3) == 0) dst->bsums[lane >> 2] = (int16_t)s16;
    if (lane < 6) dw[296 / 4 + lane] = 0;
    if (lane == 0) {
        dst->d = 1.f / iscale;
        dst->sum = total;
    }
}

__global__ __launch_bounds__(64) void k_quantize_q8k(const float* x, int ldx, HyQ8K* act, int nb) {
    const int b = blockIdx.x, t = blockIdx.y;
    q8k_quantize_wave(x + (size_t)t * ldx + (size_t)b * HY_QK, act + (size_t)t * nb + b, threadIdx.x);
}

__global__ __launch_bounds__(64) void k_quantize_q8k_pipe(PipeQuant J) {
    const int b = blockIdx.x, row = blockIdx.y;
    const int j = pipe_job(J.row0, J.njobs, row), t = row - J.row0[j], nb = J.K / HY_QK;
    q8k_quantize_wave(J.x[j] + (size_t)t * J.ldx + (size_t)b * HY_QK, J.act[j] + (size_t)t * nb + b, threadIdx.x);
}

hipError_t launch_quantize_q8k(const float* x, int ldx, HyQ8K* act, int K, int nt, hipStream_t s) {
    const int nb = K / HY_QK;
    k_quantize_q8k<<<dim3(nb, nt), 64, 0, s>>>(x, ldx, act, nb);
    return hipGetLastError();
}

hipError_t launch_quantize_q8k(const PipeQuant& J, int rows, hipStream_t s) {
    if (J.njobs < 1 || J.njobs > kPipeMax || J.K % HY_QK || rows < 1) return hipErrorInvalidValue;
    k_quantize_q8k_pipe<<<dim3(J.K / HY_QK, rows), 64, 0, s>>>(J);
    return hipGetLastError();
}

// =========================================================================== RMSNorm

// x (LDS, K floats, complete before the call) <- x * (1/sqrtf(sum(x*x)/K + eps)) * w, the
// scalar RMSNorm of src/model.c:719-739. Wavefront 0 forms the sequential sum of squares in
// index order: the exact segmented form for K <= 2048, else the squares (sq: K floats of LDS
// scratch) summed by the lane-serial chain.
__device__ void rmsnorm_lds(float* xs, float* sq, const float* w, int K, float eps, float* scale_slot) {
    if (K <= 2048) {
        if (threadIdx.x < 64) {
            const float sum = hy_wave_exact_sq_sum(xs, K, threadIdx.x);
            if (threadIdx.x == 0) *scale_slot = 1.0f / sqrtf(sum / (float)K + eps);
        }
    } else {
        for (int i = threadIdx.x; i < K; i += blockDim.x) sq[i] = xs[i] * xs[i];
        __syncthreads();
        if (threadIdx.x < 64) {
            const float sum = hy_wave_seq_sum(sq, K, threadIdx.x);
            if (threadIdx.x == 0) *scale_slot = 1.0f / sqrtf(sum / (float)K + eps);
        }
    }
    __syncthreads();
    const float scale = *scale_slot;
    for (int i = threadIdx.x; i < K; i += blockDim.x) xs[i] = xs[i] * scale * w[i];
    __syncthreads();
}

__device__ void load_vec_lds(float* xs, const float* x, int K) {
    for (int i = threadIdx.x; i < K / 4; i += blockDim.x)
        reinterpret_cast<float4*>(xs)[i] = reinterpret_cast<const float4*>(x)[i];
    __syncthreads();
}

__device__ void quantize_lds_blocks(const float* xs, HyQ8K* act, int K) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int b = wave; b < K / HY_QK; b += nw) q8k_quantize_wave(xs + b * HY_QK, act + b, lane);
}

// H = 2048, Q8_K output only: the decode matvec's prologue per token. Lane l of wavefront w
// holds values 512 w + 8 l .. + 8: the workgroup-wide exact sum of squares, x * scale * w, then
// each wavefront quantizes its two blocks.
__device__ __forceinline__ void rmsnorm_q8k_2048_row(const float* hrow, const float* w, float eps, HyQ8K* act_row) {
    __shared__ HyExactLds ex;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int off = 512 * wave + 8 * lane;
    const float* x = hrow + off;
    const float4 a0 = *reinterpret_cast<const float4*>(x), a1 = *reinterpret_cast<const float4*>(x + 4);
    const float4 u0 = *reinterpret_cast<const float4*>(w + off), u1 = *reinterpret_cast<const float4*>(w + off + 4);
    float e[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    const float nw[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    const float sum = hy_block_exact_sq_sum8<4>(e, ex, wave, lane);
    const float scale = 1.0f / sqrtf(sum / 2048.0f + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) e[i] = e[i] * scale * nw[i];
    q8k_quantize_halves(e, act_row + 2 * wave, lane);
}

__global__ __launch_bounds__(256) void k_rmsnorm_q8k_2048(const float* h, const float* w, float eps,
                                                          HyQ8K* act_out) {
    const int t = blockIdx.x;
    rmsnorm_q8k_2048_row(h + (size_t)t * 2048, w, eps, act_out + (size_t)t * 8);
}

__global__ __launch_bounds__(256) void k_rmsnorm_q8k_2048_pipe(PipeNorm J) {
    const int row = blockIdx.x, j = pipe_job(J.row0, J.njobs, row), t = row - J.row0[j];
    rmsnorm_q8k_2048_row(J.h[j] + (size_t)t * 2048, J.w[j], J.eps, J.act[j] + (size_t)t * 8);
}

__global__ __launch_bounds__(256) void k_rmsnorm_q8k(const float* h, const float* w, float eps, int H,
                                                     float* xn_out, HyQ8K* act_out) {
    extern __shared__ __align__(16) float xs[];  // [H] values, [H] squares
    __shared__ float scale_slot;
    const int t = blockIdx.x;
    load_vec_lds(xs, h + (size_t)t * H, H);
    rmsnorm_lds(xs, xs + H, w, H, eps, &scale_slot);
    if (xn_out)
        for (int i = threadIdx.x; i < H; i += blockDim.x) xn_out[(size_t)t * H + i] = xs[i];
    if (act_out) quantize_lds_blocks(xs, act_out + (size_t)t * (H / HY_QK), H);
}

hipError_t launch_rmsnorm_q8k(const PipeNorm& J, int rows, hipStream_t s) {
    if (J.njobs < 1 || J.njobs > kPipeMax || rows < 1) return hipErrorInvalidValue;
    k_rmsnorm_q8k_2048_pipe<<<rows, 256, 0, s>>>(J);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_q8k(const float* h, const float* w, float eps, int H, int nt, float* xn_out,
                              HyQ8K* act_out, hipStream_t s) {
    if (H == 2048 && !xn_out && act_out) k_rmsnorm_q8k_2048<<<nt, 256, 0, s>>>(h, w, eps, act_out);
    else k_rmsnorm_q8k<<<nt, 256, (2 * H) * sizeof(float), s>>>(h, w, eps, H, xn_out, act_out);
    return hipGetLastError();
}

// =========================================================================== matvec

int mv_segments_per_block(int kind) { return kind == KIND_PANEL ? 4 : 8; }

// Exact integer part of one 16-byte segment, reduced over the lanes of its block.
struct SegLoad {
    uint4 a;      // panel codes / Q4_K qs / Q6_K ql
    uint4 b;      // Q4_K header (d, dmin, scales) / Q6_K qh
    int sc;       // Q6_K two int8 scales packed
    uint16_t dh;  // Q6_K f16 d
};

// Segment f of a tile -> (row in tile, block, 16-byte segment of the block). spr = nb * spb
// segments per row, rcp = 1.0f / spr (both uniform): the float quotient is off by at most one
// for f < 2^24 and is corrected exactly, avoiding an integer division.
__device__ __forceinline__ void seg_coords(int spb_log2, int spr, float rcp, int f, int& rl, int& b, int& sub) {
    int q = (int)((float)f * rcp);
    int r = f - q * spr;
    if (r < 0) {
        q--;
        r += spr;
    } else if (r >= spr) {
        q++;
        r -= spr;
    }
    rl = q;
    b = r >> spb_log2;
    sub = r & ((1 << spb_log2) - 1);
}

__device__ __forceinline__ SegLoad seg_load(const MvWeight W, int kind, int row, int b, int sub) {
    SegLoad L;
    const size_t blk = (size_t)row * W.nb + b;
    if (kind == KIND_PANEL) {
        L.a = *reinterpret_cast<const uint4*>(W.w + blk * 64 + sub * 16);
    } else if (kind == KIND_Q4K) {
        const uint8_t* base = W.w + blk * 144;
        L.b = *reinterpret_cast<const uint4*>(base);
        L.a = *reinterpret_cast<const uint4*>(base + 16 + sub * 16);
    } else {  // Q6K planes: sub = h*4 + qpair*2 + lq
        const int h = sub >> 2, qpair = (sub >> 1) & 1, lq = sub & 1;
        L.a = *reinterpret_cast<const uint4*>(W.w + blk * 128 + 64 * h + 32 * qpair + 16 * lq);
        L.b = *reinterpret_cast<const uint4*>(W.w2 + blk * 64 + 32 * h + 16 * lq);
        const int j1 = 8 * h + 2 * qpair + lq;
        const int8_t* sc = W.sc + blk * 16;
        L.sc = (int)(uint8_t)sc[j1] | ((int)(uint8_t)sc[j1 + 4] << 8);
        L.dh = W.dh[blk];
    }
    return L;
}

// 6-bit scale and min j (0..7) of a Q4_K block (src/kernels.c:839-842), from the header words
// y, z, w (bytes 4..15) with variable shifts of fixed words, so the header stays in registers.
__device__ __forceinline__ int q4_scale(const uint4& hdr, int j) {
    const int lo = (int)((hdr.y >> (8 * (j & 3))) & 63u);
    const int hi = (int)(((hdr.w >> (8 * (j & 3))) & 0xFu) | (((hdr.y >> (8 * (j & 3) + 6)) & 3u) << 4));
    return j < 4 ? lo : hi;
}
__device__ __forceinline__ int q4_min(const uint4& hdr, int j) {
    const int lo = (int)((hdr.z >> (8 * (j & 3))) & 63u);
    const int hi = (int)(((hdr.w >> (8 * (j & 3) + 4)) & 0xFu) | (((hdr.z >> (8 * (j & 3) + 6)) & 3u) << 4));
    return j < 4 ? lo : hi;
}

// fp32 block term of one segment group (valid in every lane of the group). Lanes of invalid
// segments pass zeros and still join the group reductions.
template <int KIND>
__device__ __forceinline__ float seg_term(int pshift, int poff, float ps, const SegLoad L, const HyQ8K* y, int sub,
                                          bool valid) {
    if (KIND == KIND_PANEL) {
        int p = 0;
        if (valid) {
            const uint32_t w4[4] = {L.a.x, L.a.y, L.a.z, L.a.w};
            for (int l = 0; l < 4; l++) {
                const int4 q = *reinterpret_cast<const int4*>(y->qp + l * 64 + sub * 16);
                p = hy_dot4(hy_field(w4[0], l), q.x, p);
                p = hy_dot4(hy_field(w4[1], l), q.y, p);
                p = hy_dot4(hy_field(w4[2], l), q.z, p);
                p = hy_dot4(hy_field(w4[3], l), q.w, p);
            }
        }
        const int enc = hy_quad_sum(p);
        if (!valid) return 0.f;
        // src/kernels.c:576: ps * y.d * float((enc << shift) - off * sum)
        return ps * y->d * (float)((enc << pshift) - poff * y->sum);
    } else if (KIND == KIND_Q4K) {
        int si = 0, sm = 0;
        float d = 0.f, dmin = 0.f;
        if (valid) {
            const int g = sub >> 1, half = sub & 1;
            const int4 qlo = *reinterpret_cast<const int4*>(y->qs + 64 * g + 16 * half);
            const int4 qhi = *reinterpret_cast<const int4*>(y->qs + 64 * g + 32 + 16 * half);
            const uint32_t w4[4] = {L.a.x, L.a.y, L.a.z, L.a.w};
            int s0 = 0, s1 = 0;
            s0 = hy_dot4((int)(w4[0] & 0x0F0F0F0Fu), qlo.x, s0);
            s0 = hy_dot4((int)(w4[1] & 0x0F0F0F0Fu), qlo.y, s0);
            s0 = hy_dot4((int)(w4[2] & 0x0F0F0F0Fu), qlo.z, s0);
            s0 = hy_dot4((int)(w4[3] & 0x0F0F0F0Fu), qlo.w, s0);
            s1 = hy_dot4((int)((w4[0] >> 4) & 0x0F0F0F0Fu), qhi.x, s1);
            s1 = hy_dot4((int)((w4[1] >> 4) & 0x0F0F0F0Fu), qhi.y, s1);
            s1 = hy_dot4((int)((w4[2] >> 4) & 0x0F0F0F0Fu), qhi.z, s1);
            s1 = hy_dot4((int)((w4[3] >> 4) & 0x0F0F0F0Fu), qhi.w, s1);
            si = q4_scale(L.b, 2 * g) * s0 + q4_scale(L.b, 2 * g + 1) * s1;
            sm = q4_min(L.b, sub) * (y->bsums[2 * sub] + y->bsums[2 * sub + 1]);
            d = hy_f16((uint16_t)(L.b.x & 0xffffu));
            dmin = hy_f16((uint16_t)(L.b.x >> 16));
        }
        const int sumi = hy_group_sum<8>(si);
        const int summ = hy_group_sum<8>(sm);
        if (!valid) return 0.f;
        // src/kernels.c:875: y.d * (d * float(sumi) - dmin * float(summ))
        return y->d * (d * (float)sumi - dmin * (float)summ);
    } else {  // Q6K
        int acc = 0;
        if (valid) {
            const int h = sub >> 2, qpair = (sub >> 1) & 1, lq = sub & 1;
            const int j1 = 8 * h + 2 * qpair + lq, j2 = j1 + 4;
            const int4 q1 = *reinterpret_cast<const int4*>(y->qs + 16 * j1);
            const int4 q2 = *reinterpret_cast<const int4*>(y->qs + 16 * j2);
            const uint32_t wl[4] = {L.a.x, L.a.y, L.a.z, L.a.w};
            const uint32_t wh[4] = {L.b.x, L.b.y, L.b.z, L.b.w};
            const int q1a[4] = {q1.x, q1.y, q1.z, q1.w}, q2a[4] = {q2.x, q2.y, q2.z, q2.w};
            int d1 = 0, d2 = 0;
            for (int i = 0; i < 4; i++) {
                const uint32_t lo = (wl[i] & 0x0F0F0F0Fu) | (((wh[i] >> (2 * qpair)) & 0x03030303u) << 4);
                const uint32_t hi = ((wl[i] >> 4) & 0x0F0F0F0Fu) | (((wh[i] >> (2 * qpair + 4)) & 0x03030303u) << 4);
                d1 = hy_dot4((int)lo, q1a[i], d1);
                d2 = hy_dot4((int)hi, q2a[i], d2);
            }
            const int sc1 = (int)(int8_t)(L.sc & 0xff), sc2 = (int)(int8_t)((L.sc >> 8) & 0xff);
            acc = sc1 * (d1 - 32 * y->bsums[j1]) + sc2 * (d2 - 32 * y->bsums[j2]);
        }
        const int tot = hy_group_sum<8>(acc);
        if (!valid) return 0.f;
        // src/kernels.c:833: f16(d) * y.d * float(acc)
        return hy_f16(L.dh) * y->d * (float)tot;
    }
}

// Job fields read with constant indices only: a runtime index into the by-value kernel
// argument would make the compiler copy the whole argument to scratch memory.
__device__ inline MvJob mv_job(const MvLaunch& L, int j) {
    return j == 0 ? L.job[0] : (j == 1 ? L.job[1] : L.job[2]);
}
__device__ inline MvWeight mv_weight(const MvLaunch& L, int j) { return j == 0 ? L.job[0].W : L.job[1].W; }

// KIND is the weight kind of every job of the launch, or KIND_ANY for launches that mix kinds
// (then selected per workgroup at run time, with every segment field live).
template <int NT, int SEGS, int PRO, int KIND>
__global__ __launch_bounds__(NT) void k_matvec(MvLaunch L) {
    extern __shared__ __align__(64) unsigned char smem[];
    const int tid = threadIdx.x;
    const int wg = blockIdx.x;
    int j = 0;
    if (!L.pair) {
        if (L.njobs > 1 && wg >= L.job[1].wg_begin) j = 1;
        if (L.njobs > 2 && wg >= L.job[2].wg_begin) j = 2;
    }
    const MvJob J = mv_job(L, j);
    const MvWeight W = J.W;
    const MvWeight W1 = L.job[1].W;  // the up weight in pair mode
    const int kind = KIND == KIND_ANY ? W.kind : KIND;
    const int nb = W.nb;
    const int rpw = J.rows_per_wg;
    const int r0 = (wg - J.wg_begin) * rpw;
    const int rows = min(rpw, W.n - r0);
    const int spb = kind == KIND_PANEL ? 4 : 8;
    const int spb_log2 = kind == KIND_PANEL ? 2 : 3;
    const int spr = nb * spb;
    const float rcp = 1.0f / (float)spr;
    const int per_w = rows * spr;                // segments of one weight in this tile
    const int nseg = per_w * (L.pair ? 2 : 1);

    // 1. issue all weight loads of this thread first: they stay in flight through the prologue
    SegLoad ld[SEGS];
#pragma unroll
    for (int s = 0; s < SEGS; s++) {
        const int f = tid + NT * s;
        if (f < nseg) {
            const int which = L.pair ? (f >= per_w) : 0;
            int rl, b, sub;
            seg_coords(spb_log2, spr, rcp, f - which * per_w, rl, b, sub);
            ld[s] = seg_load(which ? W1 : W, kind, r0 + rl, b, sub);
        }
    }

    // 2. activation block source (the prologue builds it in LDS)
    const HyQ8K* act = L.act;
    unsigned char* terms_base = smem;
    __shared__ float scale_slot;
    if (PRO == PRO_NORM) {
        HyQ8K* act_lds = reinterpret_cast<HyQ8K*>(smem);
        float* xs = reinterpret_cast<float*>(smem + (size_t)nb * sizeof(HyQ8K));
        load_vec_lds(xs, L.x, L.K);
        rmsnorm_lds(xs, xs + L.K, L.norm_w, L.K, L.eps, &scale_slot);
        quantize_lds_blocks(xs, act_lds, L.K);
        __syncthreads();
        act = act_lds;
        terms_base = smem + (size_t)nb * sizeof(HyQ8K) + (2 * (size_t)L.K) * sizeof(float);
    } else if (PRO == PRO_QUANT) {  // quantize the fp32 input (one token) straight from global memory
        HyQ8K* act_lds = reinterpret_cast<HyQ8K*>(smem);
        quantize_lds_blocks(L.x, act_lds, L.K);
        __syncthreads();
        act = act_lds;
        terms_base = smem + (size_t)nb * sizeof(HyQ8K);
    }
    float* terms = reinterpret_cast<float*>(terms_base);  // [which][t][rl][b]

    // 3. exact block terms
    for (int t = 0; t < L.nt; t++) {
#pragma unroll
        for (int s = 0; s < SEGS; s++) {
            if (NT * s < nseg) {  // uniform: some thread of this WG has segment s
                const int f = tid + NT * s;
                const bool valid = f < nseg;
                int which = 0, rl = 0, b = 0, sub = f & (spb - 1);
                if (valid) {
                    which = L.pair ? (f >= per_w) : 0;
                    seg_coords(spb_log2, spr, rcp, f - which * per_w, rl, b, sub);
                }
                const int psh = which ? W1.pshift : W.pshift, pof = which ? W1.poff : W.poff;
                const HyQ8K* y = act + (size_t)t * nb + b;
                float term;
                if (kind == KIND_PANEL) {
                    const float* psp = which ? W1.ps : W.ps;
                    const float ps = valid && sub == 0 ? psp[(size_t)(r0 + rl) * nb + b] : 0.f;
                    term = seg_term<KIND_PANEL>(psh, pof, ps, ld[s], y, sub, valid);
                } else if (kind == KIND_Q4K) {
                    term = seg_term<KIND_Q4K>(psh, pof, 0.f, ld[s], y, sub, valid);
                } else {
                    term = seg_term<KIND_Q6K>(psh, pof, 0.f, ld[s], y, sub, valid);
                }
                if (valid && sub == 0) terms[(((size_t)which * L.nt + t) * rpw + rl) * nb + b] = term;
            }
        }
    }
    __syncthreads();

    // 4. sequential per-row combine in block order, then the epilogue
    for (int i = tid; i < rows * L.nt; i += NT) {
        const int t = i / rows, rl = i % rows;
        const float* tg = terms + ((size_t)t * rpw + rl) * nb;
        float acc = 0.f;
        for (int b = 0; b < nb; b++) acc += tg[b];
        const size_t o = (size_t)t * J.ldo + r0 + rl;
        float y;
        if (L.pair) {
            const float* tu = terms + (((size_t)L.nt + t) * rpw + rl) * nb;
            float u = 0.f;
            for (int b = 0; b < nb; b++) u += tu[b];
            // SwiGLU, src/model.c:873-876: g / (1 + expf(-g)) * u
            y = acc / (1.0f + hy_expf(-acc)) * u;
        } else if (J.epi == EPI_ADD) {
            y = J.out[o] + acc;  // residual h += tmp, src/model.c:865-869
        } else {
            y = acc;
        }
        J.out[o] = y;
    }
}

template <int NT, int PRO, int KIND>
static hipError_t launch_mv_kind(const MvLaunch& L, int grid, size_t lds, hipStream_t s) {
    switch (L.segs) {
    case 1: k_matvec<NT, 1, PRO, KIND><<<grid, NT, lds, s>>>(L); break;
    case 2: k_matvec<NT, 2, PRO, KIND><<<grid, NT, lds, s>>>(L); break;
    case 4: k_matvec<NT, 4, PRO, KIND><<<grid, NT, lds, s>>>(L); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int NT, int PRO>
static hipError_t launch_mv_nt(const MvLaunch& L, int grid, size_t lds, hipStream_t s) {
    int kind = L.job[0].W.kind;
    for (int j = 1; j < L.njobs; j++)
        if (L.job[j].W.kind != kind) kind = KIND_ANY;
    switch (kind) {
    case KIND_PANEL: return launch_mv_kind<NT, PRO, KIND_PANEL>(L, grid, lds, s);
    case KIND_Q4K: return launch_mv_kind<NT, PRO, KIND_Q4K>(L, grid, lds, s);
    case KIND_Q6K: return launch_mv_kind<NT, PRO, KIND_Q6K>(L, grid, lds, s);
    default: return launch_mv_kind<NT, PRO, KIND_ANY>(L, grid, lds, s);
    }
}

size_t matvec_lds_bytes(const MvLaunch& L, int pro) {
    int max_rpw = 0;
    for (int j = 0; j < L.njobs; j++) max_rpw = max(max_rpw, L.job[j].rows_per_wg);
    const int nb = L.job[0].W.nb;
    size_t lds = (size_t)(L.pair ? 2 : 1) * L.nt * max_rpw * nb * sizeof(float);
    if (pro == PRO_NORM) lds += (size_t)nb * sizeof(HyQ8K) + (2 * (size_t)L.K) * sizeof(float);
    if (pro == PRO_QUANT) lds += (size_t)nb * sizeof(HyQ8K);
    return lds;
}

hipError_t launch_matvec(const MvLaunch& L, int pro, int grid, hipStream_t s) {
    const size_t lds = matvec_lds_bytes(L, pro);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    if (pro != PRO_NONE && L.nt != 1) return hipErrorInvalidValue;
    if (L.threads == 1024) {
        if (pro == PRO_NORM) return launch_mv_nt<1024, PRO_NORM>(L, grid, lds, s);
        if (pro == PRO_QUANT) return launch_mv_nt<1024, PRO_QUANT>(L, grid, lds, s);
        return hipErrorInvalidValue;
    }
    if (pro == PRO_NONE) return launch_mv_nt<256, PRO_NONE>(L, grid, lds, s);
    if (pro == PRO_NORM) return launch_mv_nt<256, PRO_NORM>(L, grid, lds, s);
    return hipErrorInvalidValue;
}

// =========================================================================== RoPE + q/k norm + KV

// One wavefront per (token, head-slot): slots [0, heads) are q heads, [heads, heads+kv_heads)
// are kv heads. NeoX RoPE (src/model.c:754-765), then the per-head RMSNorm (src/model.c:840-841),
// then for kv heads the bf16 RNE store of k and v at the absolute position (src/model.c:842-847).
__device__ __forceinline__ void rope_norm_store_row(const AttnArgs& a, int t, int slot) {
    __shared__ __align__(16) float row[256];
    __shared__ __align__(16) float sq[256];
    __shared__ float scale_slot;
    const int lane = threadIdx.x;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos0) + t;
    const int hd = a.hdim, half = a.rope_half;
    const bool is_q = slot < a.heads;
    const int head = is_q ? slot : slot - a.heads;
    const int qdim = a.heads * hd, kvdim = a.kv_heads * hd;
    const float* src = is_q ? a.q + (size_t)t * qdim + (size_t)head * hd : a.k + (size_t)t * kvdim + (size_t)head * hd;
    const float* c = a.rope_cos + (size_t)pos * half;
    const float* sn = a.rope_sin + (size_t)pos * half;
    const float* nw = is_q ? a.q_norm : a.k_norm;
    const float* v = a.v + (size_t)t * kvdim + (size_t)head * hd;
    // every global operand of the row up front (dimensions lane + 64 k), so the kernel waits on
    // memory once rather than once per phase
    float xs[4], ws[4], vs[4], cs[2], ss[2];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int d = lane + 64 * k;
        xs[k] = ws[k] = vs[k] = 0.f;
        if (d < hd) {
            xs[k] = src[d];
            ws[k] = nw[d];
            if (!is_q) vs[k] = v[d];
        }
    }
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = lane + 64 * k;
        cs[k] = ss[k] = 0.f;
        if (i < half) cs[k] = c[i], ss[k] = sn[i];
    }
#pragma unroll
    for (int k = 0; k < 4; k++)
        if (lane + 64 * k < hd) row[lane + 64 * k] = xs[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = lane + 64 * k;
        if (i < half) {
            const float x0 = row[i], x1 = row[i + half];
            row[i] = x0 * cs[k] - x1 * ss[k];
            row[i + half] = x0 * ss[k] + x1 * cs[k];
        }
    }
    __syncthreads();
    for (int d = lane; d < hd; d += 64) sq[d] = row[d] * row[d];
    __syncthreads();
    {
        const float sum = hy_wave_seq_sum(sq, hd, lane);
        if (lane == 0) scale_slot = 1.0f / sqrtf(sum / (float)hd + a.eps);
    }
    __syncthreads();
    const float scale = scale_slot;
    if (is_q) {
        float* dst = a.q + (size_t)t * qdim + (size_t)head * hd;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (lane + 64 * k < hd) dst[lane + 64 * k] = row[lane + 64 * k] * scale * ws[k];
    } else {
        const size_t off = ((size_t)head * a.ctx + pos) * hd;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int d = lane + 64 * k;
            if (d < hd) {
                a.kc[off + d] = hy_to_bf16(row[d] * scale * ws[k]);
                a.vc[off + d] = hy_to_bf16(vs[k]);
            }
        }
    }
}

__global__ __launch_bounds__(64) void k_rope_norm_store(AttnArgs a) { rope_norm_store_row(a, blockIdx.x, blockIdx.y); }

__global__ __launch_bounds__(64) void k_rope_norm_store_pipe(PipeAttn J) {
    const int row = blockIdx.x, j = pipe_job(J.row0, J.njobs, row);
    rope_norm_store_row(J.a[j], row - J.row0[j], blockIdx.y);
}

hipError_t launch_rope_norm_store(const AttnArgs& a, hipStream_t s) {
    if (a.hdim > 256 || a.hdim % 4 || 2 * a.rope_half > a.hdim) return hipErrorInvalidValue;
    k_rope_norm_store<<<dim3(a.nt, a.heads + a.kv_heads), 64, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_rope_norm_store(const PipeAttn& J, int rows, hipStream_t s) {
    if (J.njobs < 1 || J.njobs > kPipeMax || rows < 1) return hipErrorInvalidValue;
    const AttnArgs& a = J.a[0];
    for (int j = 1; j < J.njobs; j++)
        if (J.a[j].heads != a.heads || J.a[j].kv_heads != a.kv_heads || J.a[j].hdim != a.hdim) return hipErrorInvalidValue;
    if (a.hdim > 256 || a.hdim % 4 || 2 * a.rope_half > a.hdim) return hipErrorInvalidValue;
    k_rope_norm_store_pipe<<<dim3(rows, a.heads + a.kv_heads), 64, 0, s>>>(J);
    return hipGetLastError();
}

// =========================================================================== attention

__device__ __forceinline__ void bf16x8(const uint4& v, float* f) {
    f[0] = hy_bitsf(v.x << 16); f[1] = hy_bitsf(v.x & 0xffff0000u);
    f[2] = hy_bitsf(v.y << 16); f[3] = hy_bitsf(v.y & 0xffff0000u);
    f[4] = hy_bitsf(v.z << 16); f[5] = hy_bitsf(v.z & 0xffff0000u);
    f[6] = hy_bitsf(v.w << 16); f[7] = hy_bitsf(v.w & 0xffff0000u);
}

// Sequential accumulation o[i] += p[j] * bf16(V[j][d0 + i]) over j in [0, cnt), V rows of hd
// bf16 values in LDS. Loads run 8 positions ahead of the dependent adds.
template <int DPL>
__device__ __forceinline__ void v_accumulate(float* o, const float* p, const uint16_t* V, int hd, int d0, int cnt) {
    int j = 0;
    for (; j + 8 <= cnt; j += 8) {
        float pj[8], vf[8][DPL];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            pj[k] = p[j + k];
            const uint16_t* vr = V + (size_t)(j + k) * hd + d0;
            if (DPL == 2) {
                const uint32_t v2 = *reinterpret_cast<const uint32_t*>(vr);
                vf[k][0] = hy_bitsf(v2 << 16);
                vf[k][DPL - 1] = hy_bitsf(v2 & 0xffff0000u);
            } else {
#pragma unroll
                for (int i = 0; i < DPL; i++) vf[k][i] = hy_bf16(vr[i]);
            }
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int i = 0; i < DPL; i++) o[i] += pj[k] * vf[k][i];
    }
    for (; j < cnt; j++) {
        const float pj = p[j];
        const uint16_t* vr = V + (size_t)j * hd + d0;
#pragma unroll
        for (int i = 0; i < DPL; i++) o[i] += pj * hy_bf16(vr[i]);
    }
}

// General attention (any nt): one workgroup per (token, q head), the reference's attn_task
// (src/model.c:767-795) with dot_bf16_scalar (src/kernels.c:1111-1121) and axpy_bf16_scalar
// (:1122-1124). Scores live in LDS; the softmax sum and the output accumulation run
// sequentially over positions. K/V of the chunk were stored by k_rope_norm_store.
template <int DPL>
__global__ __launch_bounds__(256) void k_attention(AttnArgs a) {
    extern __shared__ __align__(16) float sm[];
    __shared__ float red[8];
    const int t = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hd = a.hdim;
    const int pos = (a.pos_dev ? *a.pos_dev : a.pos0) + t;
    const int n = pos + 1;
    const int kvh = h / (a.heads / a.kv_heads);
    const int qdim = a.heads * hd;
    float* qs = sm;          // [hd]
    float* sc = sm + 256;    // [n]
    for (int d = tid; d < hd; d += 256) qs[d] = a.q[(size_t)t * qdim + (size_t)h * hd + d];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)hd);
    const uint16_t* K = a.kc + (size_t)kvh * a.ctx * hd;
    const uint16_t* V = a.vc + (size_t)kvh * a.ctx * hd;
    float mx = -__builtin_inff();
    for (int jj = tid; jj < n; jj += 256) {
        const uint16_t* kr = K + (size_t)jj * hd;
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        for (int d = 0; d < hd; d += 8) {
            float kf[8];
            bf16x8(*reinterpret_cast<const uint4*>(kr + d), kf);
            a0 += qs[d + 0] * kf[0];
            a1 += qs[d + 1] * kf[1];
            a2 += qs[d + 2] * kf[2];
            a3 += qs[d + 3] * kf[3];
            a0 += qs[d + 4] * kf[4];
            a1 += qs[d + 5] * kf[5];
            a2 += qs[d + 6] * kf[6];
            a3 += qs[d + 7] * kf[7];
        }
        const float s = ((a0 + a1) + (a2 + a3)) * scale;
        sc[jj] = s;
        mx = fmaxf(mx, s);
    }
    mx = hy_wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int jj = tid; jj < n; jj += 256) sc[jj] = hy_expf(sc[jj] - mx);
    __syncthreads();
    if (wave == 0) {
        const float sum = hy_wave_seq_sum(sc, n, lane);
        if (lane == 0) red[4] = 1.0f / sum;
    }
    __syncthreads();
    const float inv = red[4];
    for (int jj = tid; jj < n; jj += 256) sc[jj] = sc[jj] * inv;
    __syncthreads();
    if (wave == 0) {
        float o[DPL];
#pragma unroll
        for (int i = 0; i < DPL; i++) o[i] = 0.f;
        const int d0 = lane * DPL;
        v_accumulate<DPL>(o, sc, V, hd, d0, n);
        float* dst = a.ao + (size_t)t * qdim + (size_t)h * hd + d0;
#pragma unroll
        for (int i = 0; i < DPL; i++) dst[i] = o[i];
    }
}

// Chunk attention (nt tokens at consecutive positions, causal): one 512-thread workgroup per
// (KV head, token) computes the GRP query heads that share the KV head, so each K row and V
// tile is read and converted once for all of them. The arithmetic is attn_task's
// (src/model.c:767-795) per (token, head): scores by dot_bf16's four partial sums in order
// (src/kernels.c:1111-1121) times 1/sqrtf(hd), max, expf, the sum in position order,
// p_j = e_j * (1 / sum) once per position, then o[d] += p_j * V_j[d] in position order
// (axpy_bf16, :1122-1124). Scores: one key per thread for every head of the group. Sums: one
// 16-lane row of wavefront 0 per head. Output: the chains of two heads at one dimension per lane, over fp32
// V tiles in LDS.
constexpr int kAcThreads = 512;
constexpr int kAcMaxCtx = 2048;
// positions per fp32 V tile in LDS: 64 for a launch of one chunk (two workgroups a CU at any
// tile size); 32 for the pipelined launch, whose 51 KB of LDS and 74 VGPRs let three of its
// workgroups share a CU (config-4 prefill, with two heads a lane: 73.0-73.6k -> 79.2-80.1k
// tok/s; the same tile in the one-chunk launch measured 1 % slower)
constexpr int kAcTileRow = 64;
constexpr int kAcTilePipe = 32;
// output chains per lane: two heads of the group at one dimension, so each V element read from
// LDS serves both (one head a lane measured 1 % slower, four 3 % slower)
constexpr int kAcHeadsPerLane = 2;

typedef unsigned v4u __attribute__((ext_vector_type(4)));  // arrays of it stay in registers

template <int HD, int GRP, int TILE>
__device__ __forceinline__ void attn_chunk_row(const AttnArgs& a, int g, int t) {
    constexpr int NW = kAcThreads / 64;
    constexpr int KV4 = HD / 8;
    constexpr int DW = HD / 64;              // wavefronts per head in the output (one dim per lane)
    static_assert(GRP * DW <= NW && GRP <= NW, "heads x dims fit the workgroup");
    constexpr int VPC = TILE * KV4;                           // 16-byte V pieces of a tile
    constexpr int VPT = (VPC + kAcThreads - 1) / kAcThreads;  // per thread
    __shared__ __align__(16) float sc[GRP][kAcMaxCtx];   // scores, then e_j, then p_j
    __shared__ __align__(16) float vt[TILE * HD];        // fp32 V tile [j][d]
    __shared__ float red[GRP][NW];
    __shared__ float inv_s[GRP];
    __shared__ uint64_t etab[32];  // expf table (a lookup is an LDS read, not a global load)

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // uniform (read through a pointer it would count as per-lane, and so would every loop bound
    // derived from it)
    const int pos = __builtin_amdgcn_readfirstlane((a.pos_dev ? *a.pos_dev : a.pos0) + t);
    const int n = pos + 1;
    const int qdim = a.heads * HD;
    const uint16_t* K = a.kc + (size_t)g * a.ctx * HD;
    const uint16_t* V = a.vc + (size_t)g * a.ctx * HD;

    // q rows of the group's heads (RoPE'd and normed by k_rope_norm_store), read through the
    // constant address space: their addresses are uniform, so the reads are scalar loads into
    // SGPRs that the multiplies take directly (nothing is written to them in this kernel)
    if (tid < 32) etab[tid] = hy_exp_tab_entry(tid);  // read after the barrier past the scores
    typedef __attribute__((address_space(4))) const float cfloat;
    const uint64_t qaddr = (uint64_t)(uintptr_t)(a.q + (size_t)t * qdim + (size_t)(g * GRP) * HD);
    // first V tile
    v4u vr[VPT];
#pragma unroll
    for (int i = 0; i < VPT; i++) {
        const int f = tid + kAcThreads * i, j = f / KV4;
        if (VPC % kAcThreads == 0 || f < VPC) vr[i] = *reinterpret_cast<const v4u*>(V + (size_t)min(j, pos) * HD + 8 * (f % KV4));
    }
    __syncthreads();

    // scores of key j = tid + 512 p for every head
    const float scale = 1.0f / sqrtf((float)HD);
    float lmax[GRP];
#pragma unroll
    for (int h = 0; h < GRP; h++) lmax[h] = -__builtin_inff();
    for (int j = tid; j < n; j += kAcThreads) {
        const uint16_t* kr = K + (size_t)j * HD;
        uint64_t qa = qaddr;
        asm volatile("" : "+s"(qa));  // q is loaded per key, not held (or spilled) across keys
        const cfloat* qc = (const cfloat*)qa;
        float acc[GRP][4];
#pragma unroll
        for (int h = 0; h < GRP; h++) acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.f;
#pragma unroll
        for (int i = 0; i < KV4; i++) {
            const v4u kv = *reinterpret_cast<const v4u*>(kr + 8 * i);
            const float kf[8] = {hy_bitsf(kv.x << 16), hy_bitsf(kv.x & 0xffff0000u), hy_bitsf(kv.y << 16),
                                 hy_bitsf(kv.y & 0xffff0000u), hy_bitsf(kv.z << 16), hy_bitsf(kv.z & 0xffff0000u),
                                 hy_bitsf(kv.w << 16), hy_bitsf(kv.w & 0xffff0000u)};
#pragma unroll
            for (int h = 0; h < GRP; h++) {
                const cfloat* qh = qc + h * HD + 8 * i;
#pragma unroll
                for (int c = 0; c < 8; c++) acc[h][c & 3] += qh[c] * kf[c];
            }
        }
#pragma unroll
        for (int h = 0; h < GRP; h++) {
            const float sj = ((acc[h][0] + acc[h][1]) + (acc[h][2] + acc[h][3])) * scale;
            sc[h][j] = sj;
            lmax[h] = fmaxf(lmax[h], sj);
        }
    }
#pragma unroll
    for (int h = 0; h < GRP; h++) {
        const float m = hy_wave_max(lmax[h]);
        if (lane == 0) red[h][wave] = m;
    }
    __syncthreads();
    // e_j = expf(s_j - max) per head
    {
        float mx[GRP];
#pragma unroll
        for (int h = 0; h < GRP; h++) {
            mx[h] = red[h][0];
#pragma unroll
            for (int w = 1; w < NW; w++) mx[h] = fmaxf(mx[h], red[h][w]);
        }
        for (int j = tid; j < n; j += kAcThreads)
#pragma unroll
            for (int h = 0; h < GRP; h++) sc[h][j] = hy_expf_tab(sc[h][j] - mx[h], etab);
    }
    __syncthreads();
    // the sums of the heads in position order, together in the 16-lane rows of wavefront 0
    // (the chain's instructions once for all heads)
    if (wave == 0) {
        float sum[4];
        hy_row_seq_sums<GRP>(&sc[0][0], kAcMaxCtx, n, lane, sum);
        if (lane == 0)
#pragma unroll
            for (int h = 0; h < GRP; h++) inv_s[h] = 1.0f / sum[h];
    }
    __syncthreads();
    // p_j = e_j * inv, once per position (sc[j] * inv)
    {
        float inv[GRP];
#pragma unroll
        for (int h = 0; h < GRP; h++) inv[h] = inv_s[h];
        for (int j = tid; j < n; j += kAcThreads)
#pragma unroll
            for (int h = 0; h < GRP; h++) sc[h][j] = sc[h][j] * inv[h];
    }
    // output chains: HPL heads from oh0 at dimension od per lane (each V element read once for
    // them), over fp32 V tiles; the next tile's loads in flight while the current one is summed
    constexpr int HPL = GRP % kAcHeadsPerLane == 0 ? kAcHeadsPerLane : 1;
    constexpr int OW = GRP / HPL * DW;  // output wavefronts
    const int oh0 = (wave / DW) * HPL, od = (wave % DW) * 64 + lane;
    float o[HPL];
#pragma unroll
    for (int hh = 0; hh < HPL; hh++) o[hh] = 0.f;
    for (int t0 = 0; t0 < n; t0 += TILE) {
        __syncthreads();  // previous tile consumed (the first time: the p_j written)
#pragma unroll
        for (int i = 0; i < VPT; i++) {
            const int f = tid + kAcThreads * i;
            if (VPC % kAcThreads != 0 && f >= VPC) break;
            float* dstv = &vt[(f / KV4) * HD + 8 * (f % KV4)];
            const v4u w = vr[i];
            *reinterpret_cast<float4*>(dstv) =
                make_float4(hy_bitsf(w.x << 16), hy_bitsf(w.x & 0xffff0000u), hy_bitsf(w.y << 16), hy_bitsf(w.y & 0xffff0000u));
            *reinterpret_cast<float4*>(dstv + 4) =
                make_float4(hy_bitsf(w.z << 16), hy_bitsf(w.z & 0xffff0000u), hy_bitsf(w.w << 16), hy_bitsf(w.w & 0xffff0000u));
        }
        if (t0 + TILE < n) {
#pragma unroll
            for (int i = 0; i < VPT; i++) {
                const int f = tid + kAcThreads * i, j = t0 + TILE + f / KV4;
                if (VPC % kAcThreads == 0 || f < VPC) vr[i] = *reinterpret_cast<const v4u*>(V + (size_t)min(j, pos) * HD + 8 * (f % KV4));
            }
        }
        __syncthreads();  // tile in LDS
        if (wave < OW) {
            const float* vd = vt + od;
            const int cnt = min(TILE, n - t0);
            int q = 0;
            for (; q + 8 <= cnt; q += 8) {
                float vv[8];
#pragma unroll
                for (int k = 0; k < 8; k++) vv[k] = vd[(q + k) * HD];
#pragma unroll
                for (int hh = 0; hh < HPL; hh++) {
                    const float* pj = sc[oh0 + hh] + t0 + q;
                    const float4 p0 = *reinterpret_cast<const float4*>(pj);
                    const float4 p1 = *reinterpret_cast<const float4*>(pj + 4);
                    const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
                    for (int k = 0; k < 8; k++) o[hh] += pv[k] * vv[k];
                }
            }
            for (; q < cnt; q++) {
                const float vq = vd[q * HD];
#pragma unroll
                for (int hh = 0; hh < HPL; hh++) o[hh] += sc[oh0 + hh][t0 + q] * vq;
            }
        }
    }
    if (wave < OW)
#pragma unroll
        for (int hh = 0; hh < HPL; hh++) a.ao[(size_t)t * qdim + (size_t)(g * GRP + oh0 + hh) * HD + od] = o[hh];
    // the group's GRP * HD outputs are whole Q8_K blocks of the row: quantize them here
    // (quantize_q8k, src/kernels.c:128-165) for the o-projection
    if constexpr (GRP * HD % HY_QK == 0) {
        if (a.act_out) {
            constexpr int NB = GRP * HD / HY_QK;
            static_assert(NB <= NW, "one wavefront per block");
            __syncthreads();  // every chain has read its last V tile
            if (wave < OW)
#pragma unroll
                for (int hh = 0; hh < HPL; hh++) vt[(oh0 + hh) * HD + od] = o[hh];
            __syncthreads();
            if (wave < NB) q8k_quantize_wave(vt + wave * HY_QK, a.act_out + (size_t)t * (qdim / HY_QK) + g * NB + wave, lane);
        }
    }
}

template <int HD, int GRP>
__global__ __launch_bounds__(kAcThreads) void k_attn_chunk(AttnArgs a) {
    attn_chunk_row<HD, GRP, kAcTileRow>(a, blockIdx.x, blockIdx.y);
}

// Rows run last to first: the jobs are chunks in position order, so the workgroups with the
// longest rows start first and the short ones fill in behind them.
template <int HD, int GRP>
__global__ __launch_bounds__(kAcThreads, 3) void k_attn_chunk_pipe(PipeAttn J) {
    const int row = (int)(gridDim.y - 1 - blockIdx.y), j = pipe_job(J.row0, J.njobs, row);
    attn_chunk_row<HD, GRP, kAcTilePipe>(J.a[j], blockIdx.x, row - J.row0[j]);
}

// Four-token chunk attention (pipelined prefill, head dim 128, four query heads a KV head): one
// 512-thread workgroup per (KV head, four consecutive tokens) computes the 16 (token, head) rows
// with the arithmetic of attn_chunk_row (src/model.c:767-795), the products on the matrix cores.
// v_mfma_f32_16x16x1f32 with a zero accumulator returns, in lane l, register r, the product
// A[16 (r / 4) + 4 (l / 16) + r % 4] * B[16 (r / 4) + l % 16] of the lanes' operands, rounded
// once, as the separately rounded product a * b (measured bit for bit over normal, denormal and
// overflowing operands; a -0 product comes back as +0, which no sum here can tell apart: each
// starts at +0, and a round-to-nearest sum that starts at +0 is never -0). Its 16 rows are the
// (token, head) rows, 4 t + h; its four blocks are
//   scores: dot_bf16's four partial sums (src/kernels.c:1111-1121): block c takes dimension
//     4 i + c, so lane l's register 4 c + h is the chain-c product of head h of token l / 16
//     with key l % 16, and the lane keeps the 16 chains of its four scores;
//   output: four consecutive positions 4 i + b, so register 4 b + h is position 4 i + b's
//     product p_j * V_j[d] of head h of token l / 16 at dimension d = 16 w + l % 16 (wavefront w),
//     added to the head's chain in position order (axpy_bf16, :1122-1124).
// A key and a V row are read once for four tokens, each MFMA leaves the VALU 16 adds (one per
// product), and all eight wavefronts carry output chains. Rows past a token's position have
// p_j = 0, whose products add nothing. The sums of e_j in position order: wavefront t < 4 takes
// token t's four rows (hy_row_seq_sums). Scores live in LDS, 16 rows of P.sstride floats.
constexpr int kA4Threads = 512;
constexpr int kA4Tok = 4;
constexpr int kA4Tile = 32;  // V positions per bf16 LDS tile (one 16-byte piece a thread)

typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f a4_products(float row_operand, float col_operand) {
    const v16f z = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_f32_16x16x1f32(row_operand, col_operand, z, 0, 0, 0);
}

struct PipeAttn4 {
    PipeAttn J;
    int grp0[kPipeMax];  // first grid row (four-token group) of each job
    int sstride;         // score row stride in LDS, floats (4 mod 32, past the longest row)
};

// One wavefront per 64 operand pairs: the 16 products a4_products returns in each lane, stored
// out[w][r][lane] (the self-check of the zero-accumulator products and their layout)
__global__ __launch_bounds__(64) void k_selftest_mfma(const float* a, const float* b, float* out, int nw) {
    const int w = blockIdx.x, l = threadIdx.x;
    if (w >= nw) return;  // uniform
    const v16f p = a4_products(a[(size_t)w * 64 + l], b[(size_t)w * 64 + l]);
#pragma unroll
    for (int r = 0; r < 16; r++) out[((size_t)w * 16 + r) * 64 + l] = p[r];
}

hipError_t launch_selftest_mfma(const float* a, const float* b, float* out, int nw, hipStream_t s) {
    if (nw < 1) return hipErrorInvalidValue;
    k_selftest_mfma<<<nw, 64, 0, s>>>(a, b, out, nw);
    return hipGetLastError();
}

size_t attn4_lds_bytes(int sstride) { return (size_t)16 * sstride * sizeof(float) + (size_t)kA4Tile * 128 * sizeof(uint16_t); }
constexpr size_t kA4MaxDynLds = 156 * 1024;  // of the CU's 160 KB, beside the kernel's static LDS

constexpr int kA4MinWorkgroups = 256;

template <int HD>
__global__ __launch_bounds__(kA4Threads) void k_attn_chunk4_pipe(PipeAttn4 P) {
    static_assert(HD == 128, "16 output dimensions a wavefront, 8 wavefronts");
    constexpr int NW = kA4Threads / 64;
    constexpr int GRP = 4;
    static_assert(kA4Tile * HD * 2 == 16 * kA4Threads && 16 * HD * 4 == kA4Tile * HD * 2,
                  "one V piece a thread; the q rows and the outputs stage in the V tile's bytes");
    extern __shared__ __align__(16) float a4_lds[];
    __shared__ float red[NW][16];
    __shared__ float rmax[16];
    __shared__ float inv_s[16];
    __shared__ uint64_t etab[32];
    const int S = P.sstride;
    float* sc = a4_lds;                                               // [16][S]: s, then e, then p
    uint16_t* vt = reinterpret_cast<uint16_t*>(a4_lds + 16 * S);      // [kA4Tile][HD] bf16

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grow = (int)(gridDim.y - 1 - blockIdx.y);  // the jobs' last (longest) groups first
    const int jb = pipe_job(P.grp0, P.J.njobs, grow);
    const AttnArgs& a = P.J.a[jb];
    const int g = blockIdx.x;
    const int t0 = (grow - P.grp0[jb]) * kA4Tok;
    const int ntv = min(kA4Tok, a.nt - t0);  // tokens of the group
    const int pos0 = a.pos0 + t0;            // position of its first token
    const int nmax = pos0 + ntv;             // keys 0 .. nmax - 1 (the last token's row)
    const int nmax4 = (nmax + 3) & ~3;
    const int qdim = a.heads * HD;
    const uint16_t* K = a.kc + (size_t)g * a.ctx * HD;
    const uint16_t* V = a.vc + (size_t)g * a.ctx * HD;

    // first V tile's piece of this thread (position tid / 16, dimensions 8 (tid % 16) ..)
    constexpr int PPR = HD / 8;  // 16-byte pieces a position
    uint4 vr = *reinterpret_cast<const uint4*>(V + (size_t)min(tid / PPR, nmax - 1) * HD + 8 * (tid % PPR));

    // q rows chain-major in the V tile's bytes: qs[row][32 c + i] = q[token row / 4][head row % 4][4 i + c]
    if (tid < 32) etab[tid] = hy_exp_tab_entry(tid);
    {
        float* qs = reinterpret_cast<float*>(vt);
        for (int e = tid; e < 16 * HD; e += kA4Threads) {
            const int row = e / HD, d = e % HD;
            const int tt = min(row / GRP, ntv - 1), h = row % GRP;
            qs[row * HD + (d & 3) * 32 + (d >> 2)] = a.q[(size_t)(t0 + tt) * qdim + (size_t)(g * GRP + h) * HD + d];
        }
    }
    __syncthreads();
    // this lane's row operands: row l % 16, chain l / 16, i = 0 .. 31
    float qa[32];
    {
        const float* qs = reinterpret_cast<const float*>(vt) + (lane & 15) * HD + (lane >> 4) * 32;
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const float4 x = *reinterpret_cast<const float4*>(qs + i);
            qa[i] = x.x, qa[i + 1] = x.y, qa[i + 2] = x.z, qa[i + 3] = x.w;
        }
    }

    // scores: wavefront w takes the 16-key batches w, w + 8, ... (uniform loop bound); lane l
    // supplies key l % 16's dimension 4 i + l / 16, picked out of the key's 16-byte piece m = i / 2
    // into the high half of a dword (the bf16 -> fp32 conversion) by a byte permute
    const float scale = 1.0f / sqrtf((float)HD);
    const uint32_t kc2 = 2u * (uint32_t)(lane >> 4);
    const uint32_t ksel = (kc2 + 1) << 24 | kc2 << 16 | 0x0c0cu;
    const int tl = lane >> 4;                     // the token of this lane's scores
    const int nl = tl < ntv ? pos0 + tl + 1 : 0;  // its row length
    float lmax[GRP];
#pragma unroll
    for (int h = 0; h < GRP; h++) lmax[h] = -__builtin_inff();
    constexpr int KPF = 3;  // 16-byte pieces of the key row loaded ahead of their use
    uint4 kv[HD / 8];
    {
        const uint4* kr0 = reinterpret_cast<const uint4*>(K + (size_t)min(wave * 16 + (lane & 15), nmax - 1) * HD);
#pragma unroll
        for (int m = 0; m < KPF; m++) kv[m] = kr0[m];
    }
    for (int kb = wave * 16; kb < nmax; kb += NW * 16) {
        const int key = kb + (lane & 15);
        const uint4* kr = reinterpret_cast<const uint4*>(K + (size_t)min(key, nmax - 1) * HD);
        const uint4* krn = reinterpret_cast<const uint4*>(K + (size_t)min(key + NW * 16, nmax - 1) * HD);
        float acc[4][GRP];  // [chain][head]
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int h = 0; h < GRP; h++) acc[c][h] = 0.f;
        v16f prev;
#pragma unroll
        for (int i = 0; i <= HD / 4; i++) {
            v16f cur;
            if (i < HD / 4) {
                const int m = i >> 1;
                if ((i & 1) == 0) {
                    if (m + KPF < HD / 8) kv[m + KPF] = kr[m + KPF];
                    else kv[m + KPF - HD / 8] = krn[m + KPF - HD / 8];
                }
                const uint4 x = kv[m];
                const uint32_t kb32 = (i & 1) ? __builtin_amdgcn_perm(x.w, x.z, ksel) : __builtin_amdgcn_perm(x.y, x.x, ksel);
                cur = a4_products(qa[i], hy_bitsf(kb32));
            }
            if (i > 0) {
                // the previous dimension's products (its MFMA ran beside this one)
#pragma unroll
                for (int c = 0; c < 4; c++)
#pragma unroll
                    for (int h = 0; h < GRP; h++) acc[c][h] += prev[4 * c + h];
#pragma unroll
                for (int c = 0; c < 4; c++) asm volatile("" : "+v"(acc[c][0]), "+v"(acc[c][1]), "+v"(acc[c][2]), "+v"(acc[c][3]));
                __builtin_amdgcn_sched_barrier(0);
            }
            prev = cur;
        }
        if (key < nl)
#pragma unroll
            for (int h = 0; h < GRP; h++) {
                const float s = ((acc[0][h] + acc[1][h]) + (acc[2][h] + acc[3][h])) * scale;
                sc[(GRP * tl + h) * S + key] = s;
                lmax[h] = fmaxf(lmax[h], s);
            }
    }
    // row maxima: over the 16 lanes of a token, then over the wavefronts
#pragma unroll
    for (int h = 0; h < GRP; h++) {
        float m = lmax[h];
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 16));
        lmax[h] = m;
    }
    if ((lane & 15) == 0)
#pragma unroll
        for (int h = 0; h < GRP; h++) red[wave][GRP * tl + h] = lmax[h];
    __syncthreads();
    if (tid < 16) {
        float m = red[0][tid];
#pragma unroll
        for (int w = 1; w < NW; w++) m = fmaxf(m, red[w][tid]);
        rmax[tid] = m;
    }
    __syncthreads();
    // e_j = expf(s_j - max) within a row, 0 from its length to nmax4
    for (int row = 0; row < 16; row++) {
        const int tt = row / GRP, n = tt < ntv ? pos0 + tt + 1 : 0;
        const float mx = rmax[row];
        for (int j = tid; j < nmax4; j += kA4Threads) sc[row * S + j] = j < n ? hy_expf_tab(sc[row * S + j] - mx, etab) : 0.f;
    }
    __syncthreads();
    // the sums in position order: wavefront t < ntv takes token t's rows
    if (wave < ntv) {
        float sum[4];
        hy_row_seq_sums<GRP>(sc + (size_t)GRP * wave * S, S, pos0 + wave + 1, lane, sum);
        if (lane == 0)
#pragma unroll
            for (int h = 0; h < GRP; h++) inv_s[GRP * wave + h] = 1.0f / sum[h];
    }
    __syncthreads();
    // p_j = e_j * inv, once per position
    for (int row = 0; row < 16; row++) {
        const int tt = row / GRP, n = tt < ntv ? pos0 + tt + 1 : 0;
        const float inv = tt < ntv ? inv_s[row] : 0.f;
        for (int j = tid; j < n; j += kA4Threads) sc[row * S + j] = sc[row * S + j] * inv;
    }

    // output: wavefront w holds dimensions 16 w .. 16 w + 15; lane l supplies p of row l % 16 at
    // position 4 i + l / 16 and V at that position and dimension 16 w + l % 16
    const int dcol = wave * 16 + (lane & 15), prow = lane & 15, pc = lane >> 4;
    const float* pr = sc + prow * S + pc;
    float o[GRP];
#pragma unroll
    for (int h = 0; h < GRP; h++) o[h] = 0.f;
    for (int tb = 0; tb < nmax4; tb += kA4Tile) {
        __syncthreads();  // the previous tile read (the first time: p written, q rows read)
        *reinterpret_cast<uint4*>(vt + (tid / PPR) * HD + 8 * (tid % PPR)) = vr;
        if (tb + kA4Tile < nmax4)
            vr = *reinterpret_cast<const uint4*>(V + (size_t)min(tb + kA4Tile + tid / PPR, nmax - 1) * HD + 8 * (tid % PPR));
        __syncthreads();
        const int cnt = min(kA4Tile, nmax4 - tb);
        const uint16_t* vc = vt + pc * HD + dcol;
        if (cnt == kA4Tile) {
            // a whole tile: every operand read at once, each MFMA issued two steps ahead of its
            // adds (a step's region may place its MFMA last: the next step does not wait on it)
            constexpr int NQ = kA4Tile / 4;
            float pa[NQ], va[NQ];
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                pa[q] = pr[tb + 4 * q];
                va[q] = hy_bitsf((uint32_t)vc[4 * q * HD] << 16);
            }
            v16f pp[NQ];
#pragma unroll
            for (int q = 0; q < NQ + 2; q++) {
                if (q < NQ) pp[q] = a4_products(pa[q], va[q]);
                if (q >= 2) {
#pragma unroll
                    for (int b = 0; b < 4; b++)
#pragma unroll
                        for (int h = 0; h < GRP; h++) o[h] += pp[q - 2][4 * b + h];
                    asm volatile("" : "+v"(o[0]), "+v"(o[1]), "+v"(o[2]), "+v"(o[3]));
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else {
            for (int i = 0; i < cnt; i += 4) {
                const v16f p = a4_products(pr[tb + i], hy_bitsf((uint32_t)vc[i * HD] << 16));
#pragma unroll
                for (int b = 0; b < 4; b++)
#pragma unroll
                    for (int h = 0; h < GRP; h++) o[h] += p[4 * b + h];
            }
        }
    }
    if (tl < ntv)
#pragma unroll
        for (int h = 0; h < GRP; h++) a.ao[(size_t)(t0 + tl) * qdim + (size_t)(g * GRP + h) * HD + dcol] = o[h];
    // each token's GRP * HD = 512 outputs are two Q8_K blocks of its row: quantize them here
    // (quantize_q8k, src/kernels.c:128-165), staged in the V tile's bytes
    if (a.act_out) {
        __syncthreads();  // every chain has read its last V tile
        float* ob = reinterpret_cast<float*>(vt);
#pragma unroll
        for (int h = 0; h < GRP; h++) ob[tl * GRP * HD + h * HD + dcol] = o[h];
        __syncthreads();
        const int tq = wave >> 1, bq = wave & 1;
        if (tq < ntv) q8k_quantize_wave(ob + tq * GRP * HD + bq * HY_QK, a.act_out + (size_t)(t0 + tq) * (qdim / HY_QK) + g * 2 + bq, lane);
    }
}

// The four-token kernel for head dim 128 with four query heads a KV head, where every job's
// positions are the host's and the rows fit in LDS; false where it does not apply.
static bool launch_attn4(const PipeAttn& J, hipStream_t s, hipError_t& err) {
    PipeAttn4 P;
    P.J = J;
    int groups = 0, nmax = 0;
    for (int j = 0; j < J.njobs; j++) {
        if (J.a[j].pos_dev) return false;
        P.grp0[j] = groups;
        groups += (J.a[j].nt + kA4Tok - 1) / kA4Tok;
        nmax = std::max(nmax, J.a[j].pos0 + J.a[j].nt);
    }
    // at least a workgroup a CU: below that (one 128-token chunk at four KV heads: 128 groups) the
    // per-token kernel's four times as many workgroups finish first (config-4 prefill one chunk
    // after another: 46.2k against 39.7k tok/s; pipelined, with 256 and more: 99k against 90k)
    if (groups * J.a[0].kv_heads < kA4MinWorkgroups) return false;
    P.sstride = ((nmax + 31) & ~31) + 4;
    const size_t lds = attn4_lds_bytes(P.sstride);
    if (lds > kA4MaxDynLds) return false;
    // the dynamic-LDS allowance, once per device (a repeat from another host thread is harmless)
    static bool attr_set[64] = {};
    int dev = 0;
    if ((err = hipGetDevice(&dev)) != hipSuccess) return true;
    if (dev < 0 || dev >= 64 || !attr_set[dev]) {
        err = hipFuncSetAttribute(reinterpret_cast<const void*>(k_attn_chunk4_pipe<128>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kA4MaxDynLds);
        if (err != hipSuccess) return true;
        if (dev >= 0 && dev < 64) attr_set[dev] = true;
    }
    k_attn_chunk4_pipe<128><<<dim3(J.a[0].kv_heads, groups), kA4Threads, lds, s>>>(P);
    err = hipGetLastError();
    return true;
}

bool attention_quantizes(const AttnArgs& a) {
    if (a.ctx > kAcMaxCtx || a.heads % a.kv_heads) return false;
    const int grp = a.heads / a.kv_heads;
    if (!((a.hdim == 128 || a.hdim == 64) && (grp == 4 || grp == 2))) return false;
    return grp * a.hdim % HY_QK == 0;
}

hipError_t launch_attention(const PipeAttn& J, int rows, hipStream_t s) {
    if (J.njobs < 1 || J.njobs > kPipeMax || rows < 1) return hipErrorInvalidValue;
    const AttnArgs& a = J.a[0];
    for (int j = 0; j < J.njobs; j++) {
        const AttnArgs& b = J.a[j];
        if (b.heads != a.heads || b.kv_heads != a.kv_heads || b.hdim != a.hdim || !b.act_out || !attention_quantizes(b))
            return hipErrorNotSupported;
    }
    const int grp = a.heads / a.kv_heads;
    if (a.hdim == 128 && grp == 4) {
        hipError_t e;
        if (launch_attn4(J, s, e)) return e;
    }
    const dim3 grid(a.kv_heads, rows);
    if (a.hdim == 128 && grp == 4) k_attn_chunk_pipe<128, 4><<<grid, kAcThreads, 0, s>>>(J);
    else if (a.hdim == 128 && grp == 2) k_attn_chunk_pipe<128, 2><<<grid, kAcThreads, 0, s>>>(J);
    else if (a.hdim == 64 && grp == 4) k_attn_chunk_pipe<64, 4><<<grid, kAcThreads, 0, s>>>(J);
    else return hipErrorNotSupported;  // head dim 64 with 2 query heads per KV head does not quantize in place
    return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t s) {
    // causal chunk attention per (KV head, token) where it applies
    int grp = a.heads % a.kv_heads == 0 ? a.heads / a.kv_heads : 0;
    if (a.ctx <= kAcMaxCtx && a.hdim == 128 && grp == 4) {
        PipeAttn J{};
        J.a[0] = a;
        J.njobs = 1;
        hipError_t e;
        if (launch_attn4(J, s, e)) return e;
    }
    if (a.ctx <= kAcMaxCtx) {
        const dim3 grid(a.kv_heads, a.nt);
        if (a.hdim == 128 && grp == 4) k_attn_chunk<128, 4><<<grid, kAcThreads, 0, s>>>(a);
        else if (a.hdim == 128 && grp == 2) k_attn_chunk<128, 2><<<grid, kAcThreads, 0, s>>>(a);
        else if (a.hdim == 64 && grp == 4) k_attn_chunk<64, 4><<<grid, kAcThreads, 0, s>>>(a);
        else if (a.hdim == 64 && grp == 2) k_attn_chunk<64, 2><<<grid, kAcThreads, 0, s>>>(a);
        else grp = 0;
        if (grp) return hipGetLastError();
    }
    const size_t lds = (256 + (size_t)a.ctx + 4) * sizeof(float);
    if (lds > 160 * 1024 || a.heads % a.kv_heads) return hipErrorInvalidValue;
    const dim3 grid(a.nt, a.heads);
    switch (a.hdim) {
    case 64: k_attention<1><<<grid, 256, lds, s>>>(a); break;
    case 128: k_attention<2><<<grid, 256, lds, s>>>(a); break;
    case 256: k_attention<4><<<grid, 256, lds, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// =========================================================================== LM head

// One lane per vocabulary row: logits[r] = sum_j w(r, j) * xn[j] accumulated sequentially in the
// reference's order, after the output RMSNorm (src/model.c:888-890):
//   F16 / F32: s += f16_to_f32(w) * x, one product and one add per weight (src/kernels.c:1279-1300)
//   Q8_0: per 32-weight block s_b = sum_j (float)q_j * x_j, then sum += f16_to_f32(d_b) * s_b
//         (dot_q8_0_f32, src/kernels.c:1099-1107)
// A workgroup owns kHeadThreads consecutive rows of one row tile (one per thread). In the
// row-tiled layout piece q (16 bytes) of the tile's rows is one contiguous 4 KB run, so every
// thread reads its own row straight into registers with coalesced loads: a stage is 64 bytes of the row (four pieces),
// and NS register sets rotate, NS - 1 stages in flight while one is summed (NS = 8 for F16 and
// F32: 32 KB in flight per wavefront keeps HBM busy with one or two workgroups per CU; 4 for
// Q8_0). Q8_0 scales come from their own row tiles, one 16-byte piece (8 blocks = 4 stages) at a
// time, a piece ahead. No LDS staging and no barriers past the norm. Optionally folds the greedy
// argmax (first index on ties, src/model.c:945-948) into one key per workgroup (slots) or a
// 64-bit atomicMax key.
template <int KIND>
__global__ __launch_bounds__(kHeadThreads) void k_head(HeadArgs a) {
    constexpr int NS = KIND == KIND_Q8_0 ? 4 : 8;
    extern __shared__ __align__(16) float xs[];    // [K] normalized input, [K] squares
    __shared__ float scale_slot;
    hy_sgpr_pin(a.W.w), hy_sgpr_pin(a.W.w2), hy_sgpr_pin(a.W.k), hy_sgpr_pin(a.W.n), hy_sgpr_pin(a.h),
        hy_sgpr_pin(a.norm_w), hy_sgpr_pin(a.eps), hy_sgpr_pin(a.logits), hy_sgpr_pin(a.argmax_key),
        hy_sgpr_pin(a.n_arg), hy_sgpr_pin(blockDim.x);
    static_assert(kRowTile % kHeadThreads == 0, "a workgroup takes whole rows of one tile");
    constexpr int SUB = kRowTile / kHeadThreads;  // workgroups per row tile
    constexpr int WB = KIND == KIND_F16 ? 2 : KIND == KIND_F32 ? 4 : 1;  // bytes per weight
    const int tid = threadIdx.x;
    const int K = a.W.k, n = a.W.n;
    const int tile = blockIdx.x / SUB, tr0 = (blockIdx.x % SUB) * kHeadThreads;  // first row in the tile
    const int r0 = tile * kRowTile + tr0;
    const int rowb = WB * K;
    const int nstage = rowb / 64;
    // piece q of this thread's row
    const uint8_t* src = a.W.w + (size_t)tile * kRowTile * rowb + (size_t)(tr0 + tid) * 16;
    // stage st = pieces 4 st .. 4 st + 3; stages past the last repeat it, unused
    auto ld = [&](v4u (&p)[4], int st) __attribute__((always_inline)) {
        const size_t c = (size_t)min(st, nstage - 1) * 4 * (kRowTile * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) p[i] = *reinterpret_cast<const v4u*>(src + c + (size_t)i * (kRowTile * 16));
    };
    // Q8_0 scales: piece g holds the f16 d of blocks 8 g .. 8 g + 7 (stages 4 g .. 4 g + 3)
    const int dpieces = K / 256;
    const uint8_t* dsrc = KIND == KIND_Q8_0 ? a.W.w2 + (size_t)tile * kRowTile * (K / 16) + (size_t)(tr0 + tid) * 16
                                            : nullptr;
    auto ld_d = [&](int g) __attribute__((always_inline)) {
        return *reinterpret_cast<const v4u*>(dsrc + (size_t)min(g, dpieces - 1) * (kRowTile * 16));
    };
    v4u dcur = {0, 0, 0, 0}, dnext = {0, 0, 0, 0};
    float acc = 0.f;
    auto comp = [&](const v4u (&p)[4], int st, int q4) __attribute__((always_inline)) {  // q4 = st % 4 (Q8_0)
        if (st >= nstage) return;
        if (KIND == KIND_F16) {
            const float* xk = xs + st * 32;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t w[4] = {p[q].x, p[q].y, p[q].z, p[q].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    acc += hy_f16((uint16_t)(w[e] & 0xffffu)) * xk[8 * q + 2 * e];
                    acc += hy_f16((uint16_t)(w[e] >> 16)) * xk[8 * q + 2 * e + 1];
                }
            }
        } else if (KIND == KIND_F32) {
            const float* xk = xs + st * 16;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                acc += hy_bitsf(p[q].x) * xk[4 * q + 0];
                acc += hy_bitsf(p[q].y) * xk[4 * q + 1];
                acc += hy_bitsf(p[q].z) * xk[4 * q + 2];
                acc += hy_bitsf(p[q].w) * xk[4 * q + 3];
            }
        } else {  // Q8_0: blocks 2 st and 2 st + 1, scales at halves (2 st) % 8 and (2 st + 1) % 8
            const float* xk = xs + st * 64;
            const uint32_t dw = q4 == 0 ? dcur.x : q4 == 1 ? dcur.y : q4 == 2 ? dcur.z : dcur.w;
#pragma unroll
            for (int blk = 0; blk < 2; blk++) {
                float sb = 0.f;
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const v4u& pc = p[2 * blk + q];
                    const uint32_t w[4] = {pc.x, pc.y, pc.z, pc.w};
#pragma unroll
                    for (int e = 0; e < 16; e++)
                        sb += (float)(int8_t)(w[e >> 2] >> (8 * (e & 3))) * xk[32 * blk + 16 * q + e];
                }
                acc += hy_f16((uint16_t)(blk ? dw >> 16 : dw & 0xffffu)) * sb;
            }
        }
    };
    load_vec_lds(xs, a.h, K);  // first: loads return in issue order
    if (KIND == KIND_Q8_0) {
        dcur = ld_d(0);
        dnext = ld_d(1);
    }
    if constexpr (KIND == KIND_Q8_0) {
        // four named register sets: an array of them, or eight, spills with the scale logic
        v4u s0[4], s1[4], s2[4], s3[4];
        ld(s0, 0);
        ld(s1, 1);
        ld(s2, 2);
        ld(s3, 3);
        rmsnorm_lds(xs, xs + K, a.norm_w, K, a.eps, &scale_slot);  // while the weights stream
        for (int st = 0; st < nstage; st += 4) {
            comp(s0, st, 0);
            ld(s0, st + 4);
            comp(s1, st + 1, 1);
            ld(s1, st + 5);
            comp(s2, st + 2, 2);
            ld(s2, st + 6);
            comp(s3, st + 3, 3);
            ld(s3, st + 7);
            dcur = dnext;
            dnext = ld_d(st / 4 + 2);
        }
    } else {
        v4u sb[NS][4];
#pragma unroll
        for (int i = 0; i < NS; i++) ld(sb[i], i);
        rmsnorm_lds(xs, xs + K, a.norm_w, K, a.eps, &scale_slot);  // while the weights stream
        for (int st = 0; st < nstage; st += NS) {
#pragma unroll
            for (int i = 0; i < NS; i++) {
                comp(sb[i], st + i, 0);
                ld(sb[i], st + NS + i);
            }
        }
    }
    const int r = r0 + tid;
    if (r < n) a.logits[r] = acc;
    if (a.slots) {
        hy_wg_slot_max(r < a.n_arg ? argmax_key(acc, r) : 0ull, a.slots + blockIdx.x);
    } else if (a.argmax_key) {
        unsigned long long key = (r < a.n_arg) ? argmax_key(acc, r) : 0ull;
        key = wave_max_u64(key);
        if ((tid & 63) == 0 && key) atomicMax(a.argmax_key, key);
    }
}

hipError_t launch_head(const HeadArgs& a, hipStream_t s) {
    const int grid = head_grid(a.W.n);
    const size_t lds = (2 * (size_t)a.W.k) * sizeof(float);
    if (a.W.kind == KIND_F16) {
        if (a.W.k % 32) return hipErrorInvalidValue;
        k_head<KIND_F16><<<grid, kHeadThreads, lds, s>>>(a);
    } else if (a.W.kind == KIND_F32) {
        if (a.W.k % 16) return hipErrorInvalidValue;
        k_head<KIND_F32><<<grid, kHeadThreads, lds, s>>>(a);
    } else if (a.W.kind == KIND_Q8_0) {
        if (a.W.k % 256) return hipErrorInvalidValue;
        k_head<KIND_Q8_0><<<grid, kHeadThreads, lds, s>>>(a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// =========================================================================== step finish

// Element i of row tok of an uploaded embedding, as the reference's dequant_row computes it
// (src/kernels.c:1304-1329): F16 / F32 / Q8_0 from their row tiles (hy_tile_offset); Q4_K from
// the raw blocks (q4_k_dequant_row, :844-859: d1 * q - m1 with d1 = d * sc, m1 = dmin * m);
// Q6_K from its planes (q6_k_dequant_row, :786-806: d * sc * (q - 32)).
__device__ float embed_elem(const MvWeight& E, int tok, int i, int H) {
    switch (E.kind) {
    case KIND_F16:
        return hy_f16(reinterpret_cast<const uint16_t*>(E.w)[hy_tile_offset(tok, 2 * (size_t)i, 2 * (size_t)H) / 2]);
    case KIND_F32:
        return reinterpret_cast<const float*>(E.w)[hy_tile_offset(tok, 4 * (size_t)i, 4 * (size_t)H) / 4];
    case KIND_Q8_0: {
        const float d = hy_f16(
            reinterpret_cast<const uint16_t*>(E.w2)[hy_tile_offset(tok, 2 * (size_t)(i / 32), (size_t)H / 16) / 2]);
        return d * (float)(int8_t)E.w[hy_tile_offset(tok, (size_t)i, (size_t)H)];
    }
    case KIND_Q4K: {
        const uint8_t* b = E.w + ((size_t)tok * E.nb + i / 256) * 144;
        const int j = i % 256, g = j / 64, is = 2 * g + ((j % 64) >= 32);
        const float d = hy_f16((uint16_t)(b[0] | (b[1] << 8))), dmin = hy_f16((uint16_t)(b[2] | (b[3] << 8)));
        const uint8_t* sc = b + 4;
        int scv, mv;
        if (is < 4) {
            scv = sc[is] & 63;
            mv = sc[is + 4] & 63;
        } else {
            scv = (sc[is + 4] & 0xF) | ((sc[is - 4] >> 6) << 4);
            mv = (sc[is + 4] >> 4) | ((sc[is] >> 6) << 4);
        }
        const uint8_t qb = b[16 + 32 * g + j % 32];
        const int q = (j % 64) < 32 ? (qb & 0xF) : (qb >> 4);
        const float d1 = d * (float)scv, m1 = dmin * (float)mv;
        return d1 * (float)q - m1;
    }
    case KIND_Q6K: {
        const size_t blk = (size_t)tok * E.nb + i / 256;
        const int j = i % 256, half = j / 128, qd = (j % 128) / 32, l = j % 32;
        const uint8_t ql = E.w[blk * 128 + half * 64 + (qd & 1) * 32 + l];
        const uint8_t qh = E.w2[blk * 64 + half * 32 + l];
        const int q = ((qd < 2) ? (ql & 0xF) : (ql >> 4)) | (((qh >> (2 * qd)) & 3) << 4);
        const float d = hy_f16(E.dh[blk]);
        return d * (float)E.sc[blk * 16 + half * 8 + l / 16 + 2 * qd] * (float)(q - 32);
    }
    default:
        return 0.f;
    }
}

// Row tok of an uploaded embedding into h (dequant_row, src/kernels.c:1304). F16 / F32 rows are
// read as whole 16-byte pieces of the row-tiled layout (piece p holds the row's bytes
// 16p .. 16p + 15); the block formats element by element.
__device__ void embed_row(const MvWeight& E, int tok, float* h, int H) {
    if (E.kind == KIND_F16 || E.kind == KIND_F32) {
        const int wb = E.kind == KIND_F16 ? 2 : 4, rowb = wb * H;
        for (int p = threadIdx.x; p < rowb / 16; p += blockDim.x) {
            const v4u q = *reinterpret_cast<const v4u*>(E.w + hy_tile_offset(tok, 16 * (size_t)p, rowb));
            float4* dst = reinterpret_cast<float4*>(h + p * (16 / wb));
            if (wb == 2) {
                dst[0] = make_float4(hy_f16((uint16_t)(q.x & 0xffffu)), hy_f16((uint16_t)(q.x >> 16)),
                                     hy_f16((uint16_t)(q.y & 0xffffu)), hy_f16((uint16_t)(q.y >> 16)));
                dst[1] = make_float4(hy_f16((uint16_t)(q.z & 0xffffu)), hy_f16((uint16_t)(q.z >> 16)),
                                     hy_f16((uint16_t)(q.w & 0xffffu)), hy_f16((uint16_t)(q.w >> 16)));
            } else {
                dst[0] = make_float4(hy_bitsf(q.x), hy_bitsf(q.y), hy_bitsf(q.z), hy_bitsf(q.w));
            }
        }
        return;
    }
    for (int i = threadIdx.x; i < H; i += blockDim.x) h[i] = embed_elem(E, tok, i, H);
}

// Greedy step tail: token = the maximum of the head's per-workgroup argmax keys; the next input
// is the next prompt id while the prompt lasts, else the argmax (recorded in ids). Embeds the
// next token's row into h, copies the next position's RoPE row and advances the device step
// counter. The step and the prompt id are read by every thread (uniform scalar loads); the slots
// are reduced over the workgroup before the embedding.
__global__ __launch_bounds__(256) void k_finish(FinishArgs a) {
    hy_sgpr_pin(a.slots), hy_sgpr_pin(a.nslots), hy_sgpr_pin(a.ids), hy_sgpr_pin(a.step), hy_sgpr_pin(a.n_prompt),
        hy_sgpr_pin(a.E.w), hy_sgpr_pin(a.E.kind), hy_sgpr_pin(a.h), hy_sgpr_pin(a.H), hy_sgpr_pin(a.n_total),
        hy_sgpr_pin(a.rope_cur), hy_sgpr_pin(a.rope_cos), hy_sgpr_pin(a.rope_sin), hy_sgpr_pin(a.rope_half),
        hy_sgpr_pin(a.ctx), hy_sgpr_pin(a.stop), hy_sgpr_pin(a.stop_host), hy_sgpr_pin(blockDim.x);
    __shared__ unsigned long long kw[4];
    // the stop ids and the first stop position (uniform: loaded with the arguments, off the
    // critical path)
    int stv[kStopIds + 1];
#pragma unroll
    for (int j = 0; j <= kStopIds; j++) stv[j] = a.stop[j];
    // the slot maxima, eight loads in flight per thread; indices past the end re-read the last
    // slot (a maximum is unchanged by repeats), so every load is unconditional
    unsigned long long key = 0ull;
    const int last = a.nslots - 1;
    for (int base = threadIdx.x; base <= last; base += 8 * 256) {
        unsigned long long v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = a.slots[min(base + 256 * u, last)];
#pragma unroll
        for (int u = 0; u < 8; u++) key = v[u] > key ? v[u] : key;
    }
    key = wave_max_u64(key);
    if ((threadIdx.x & 63) == 0) kw[threadIdx.x >> 6] = key;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 4; w++) key = kw[w] > key ? kw[w] : key;
    const int step = *a.step;
    const int nx = step + 1;
    const int pid = a.ids[min(nx, a.n_total - 1)];  // the next prompt id, if the prompt lasts
    const int best = key ? (int)(0xffffffffu - (uint32_t)(key & 0xffffffffull)) : 0;
    const int next_tok = nx < a.n_prompt ? pid : best;
    if (a.rope_cur && nx < a.ctx) {
        for (int i = threadIdx.x; i < a.rope_half; i += blockDim.x) {
            a.rope_cur[i] = a.rope_cos[(size_t)nx * a.rope_half + i];
            a.rope_cur[a.rope_half + i] = a.rope_sin[(size_t)nx * a.rope_half + i];
        }
    }
    embed_row(a.E, next_tok, a.h, a.H);
    __syncthreads();
    if (threadIdx.x == 0) {
        if (nx >= a.n_prompt && nx < a.n_total) {
            a.ids[nx] = best;
            // the reference's loop ends before a stop id (src/model.c:949); the device loop runs
            // on and only records the first position where that happened
            bool hit = false;
#pragma unroll
            for (int j = 0; j < kStopIds; j++) hit |= best == stv[j];
            if (hit && stv[kStopIds] > nx) {
                a.stop[kStopIds] = nx;
                *a.stop_host = nx;
            }
        }
        *a.step = nx;
    }
}

hipError_t launch_finish(const FinishArgs& a, hipStream_t s) {
    k_finish<<<1, 256, 0, s>>>(a);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_embed(const int* ids, const int* step, MvWeight E, float* h, int H) {
    embed_row(E, ids[*step], h, H);
}

hipError_t launch_embed(const int* ids, const int* step, const MvWeight& E, float* h, int H, hipStream_t s) {
    if (!embed_kind(E.kind)) return hipErrorInvalidValue;
    k_embed<<<1, 256, 0, s>>>(ids, step, E, h, H);
    return hipGetLastError();
}

// Embedding rows of nt consecutive ids (ids[first + t] -> h[t]), for a prefill chunk.
__global__ __launch_bounds__(256) void k_embed_rows(const int* ids, int first, MvWeight E, float* h, int H) {
    embed_row(E, ids[first + blockIdx.x], h + (size_t)blockIdx.x * H, H);
}

hipError_t launch_embed_rows(const int* ids, int first, int nt, const MvWeight& E, float* h, int H, hipStream_t s) {
    if (!embed_kind(E.kind)) return hipErrorInvalidValue;
    k_embed_rows<<<nt, 256, 0, s>>>(ids, first, E, h, H);
    return hipGetLastError();
}

__global__ void k_set_int(int* p, int v) { *p = v; }

hipError_t launch_set_int(int* p, int v, hipStream_t s) {
    k_set_int<<<1, 1, 0, s>>>(p, v);
    return hipGetLastError();
}

// =========================================================================== small kernels

// Greedy argmax over rows [0, n) of fp32 logits into a 64-bit key (first index on ties).
__global__ __launch_bounds__(256) void k_argmax(const float* v, int n, unsigned long long* slots) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    hy_wg_slot_max(i < n ? argmax_key(v[i], i) : 0ull, slots + blockIdx.x);
}

hipError_t launch_argmax(const float* v, int n, unsigned long long* slots, hipStream_t s) {
    k_argmax<<<argmax_grid(n), 256, 0, s>>>(v, n, slots);
    return hipGetLastError();
}

// g <- g / (1 + expf(-g)) * u (src/model.c:873-876), for gate/up pairs that cannot share tiles.
__global__ void k_silu_mul(float* g, const float* u, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float x = g[i];
        g[i] = x / (1.0f + hy_expf(-x)) * u[i];
    }
}

hipError_t launch_silu_mul(float* g, const float* u, int n, hipStream_t s) {
    k_silu_mul<<<(n + 255) / 256, 256, 0, s>>>(g, u, n);
    return hipGetLastError();
}

__global__ void k_selftest(const void* src, float* dst, int n, int what) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    if (what == 0) dst[i] = hy_f16(reinterpret_cast<const uint16_t*>(src)[i]);
    else dst[i] = hy_expf(reinterpret_cast<const float*>(src)[i]);
}

// One wavefront per vector: the sequential sum of squares of x[v*n .. v*n + n), by the
// lane-serial chain (method 0) or the exact segmented form (method 1).
__global__ __launch_bounds__(64) void k_selftest_sqsum(const float* x, int n, float* out, int method) {
    const float* p = x + (size_t)blockIdx.x * n;
    const float s = method ? hy_wave_exact_sq_sum(p, n, threadIdx.x) : hy_wave_seq_sq_sum(p, n, threadIdx.x);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
}

// One 256-thread workgroup per vector: the workgroup-wide exact form (method 2) the decode
// matvec's RMSNorm uses, values past n read as zero.
__global__ __launch_bounds__(256) void k_selftest_sqsum_block(const float* x, int n, float* out) {
    __shared__ HyExactLds lds;
    const float* p = x + (size_t)blockIdx.x * n;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, e0 = 512 * wave + 8 * lane;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = e0 + i < n ? p[e0 + i] : 0.f;
    const float s = hy_block_exact_sq_sum8<4>(v, lds, wave, lane);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
}

// Method 3: the plain (non-squared) sequential sum of n <= 4096 non-negative addends by the
// 8-wavefront form, as the decode attention's softmax denominator uses it.
__global__ __launch_bounds__(512) void k_selftest_sum_block8(const float* x, int n, float* out) {
    __shared__ HyExactLdsT<8> lds;
    const float* p = x + (size_t)blockIdx.x * n;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, e0 = 512 * wave + 8 * lane;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = e0 + i < n ? p[e0 + i] : 0.f;
    const float s = hy_block_exact_sum8<8, false>(v, lds, wave, lane);
    if (threadIdx.x == 0) out[blockIdx.x] = s;
}

hipError_t launch_selftest_sqsum(const float* x, int n, int m, float* out, int method, hipStream_t s) {
    if (n < 1 || (n & 3) || m < 1 || method < 0 || method > 3 || n > (method == 3 ? 4096 : 2048))
        return hipErrorInvalidValue;
    if (method == 3) k_selftest_sum_block8<<<m, 512, 0, s>>>(x, n, out);
    else if (method == 2) k_selftest_sqsum_block<<<m, 256, 0, s>>>(x, n, out);
    else k_selftest_sqsum<<<m, 64, 0, s>>>(x, n, out, method);
    return hipGetLastError();
}

hipError_t launch_selftest(const void* src, float* dst, int n, int what, hipStream_t s) {
    k_selftest<<<(n + 255) / 256, 256, 0, s>>>(src, dst, n, what);
    return hipGetLastError();
}

}  // namespace hy
