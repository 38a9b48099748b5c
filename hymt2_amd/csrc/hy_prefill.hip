// Multi-token GEMM of the panel formats (STQ1_0 and Q2_0C after the host's load-time repack)
// on int8 MFMA, gfx950: the dense contraction of chunked prefill.
//
// The reference multiplies a chunk one (row, token) pair at a time (panel_rows_scalar,
// src/kernels.c:565-581):
//   enc   = sum over the 256 positions of a block of code(0..3) * qp        (exact int32)
//   acc  += ps[r][b] * d[t][b] * (float)((enc << pshift) - poff * sum[t][b])   (fp32, block order)
// The int32 block dot is what v_mfma_i32_16x16x64_i8 computes, exactly and in any order; the
// fp32 combination then runs per (row, token) in block order, as in the reference, so the
// result is bit-identical to the single-token path.
//
// Operands. Panel byte i of a block carries the 2-bit codes of positions i, 64+i, 128+i, 192+i
// (bits 2l..2l+1 pair with qp[64 l + i]). For the K = 64 chunk l of a block, MFMA lane
// (m = lane % 16, g = lane / 16) takes A bytes j = 0..15 as code bits 2l of panel bytes 16g + j
// of row m, and B bytes as qp[64 l + 16 g + j] of token m: one 16-byte load of the row's panel
// bytes feeds all four chunks (a shift and mask per chunk), and the activation side is four
// 16-byte loads per token. C lane i holds rows 4 (i / 16) + r, r = 0..3, of token i % 16.
//
// Work layout: 256-thread workgroups of 4 wavefronts in a WR x WT grid; a wavefront owns MT
// row tiles x NT token tiles of 16 x 16. In gate/up pair mode MT = 2 and the two row tiles of a
// wavefront are the gate and up rows of the same 16 outputs, so the SwiGLU epilogue
// (src/model.c:873-876) has both values in one register. The per-row block scales of the
// workgroup's rows are staged in LDS once; everything else streams from L2 through registers,
// the next block's fragments loaded while the current block's MFMAs run.
#include "hy_kernels.h"

namespace hy {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kGemmMaxNb = 64;  // K <= 16384 (LDS for the row scales)

struct GemmFrag {
    uint4 a[2];      // panel bytes of this lane's row in each row tile
    uint4 q[2][4];   // qp chunks of this lane's token in each token tile
    float d[2];
    int sum[2];
};

__device__ __forceinline__ v4i chunk_codes(const uint4& p, int l) {
    const int sh = 2 * l;
    v4i r;
    r[0] = (int)((p.x >> sh) & 0x03030303u);
    r[1] = (int)((p.y >> sh) & 0x03030303u);
    r[2] = (int)((p.z >> sh) & 0x03030303u);
    r[3] = (int)((p.w >> sh) & 0x03030303u);
    return r;
}

__device__ __forceinline__ v4i as_v4i(const uint4& u) {
    v4i r;
    r[0] = (int)u.x;
    r[1] = (int)u.y;
    r[2] = (int)u.z;
    r[3] = (int)u.w;
    return r;
}

template <int MT, int NT, int WR, int WT, bool PAIR>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_panel(GemmLaunch L) {
    static_assert(WR * WT == kGemmThreads / 64, "4 wavefronts per workgroup");
    static_assert(!PAIR || MT == 2, "pair mode: one gate and one up tile per wavefront");
    static_assert(MT <= 2 && NT <= 2, "fragment arrays");
    constexpr int SLOTS = WR * MT * 16;  // row slots of the workgroup
    __shared__ __align__(16) float ps_lds[kGemmMaxNb * SLOTS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave % WR, wt = wave / WR;
    const int nb = L.nb, nt = L.nt;

    // job of this row tile
    int j = 0;
#pragma unroll
    for (int q = 1; q < kMaxJobs; q++)
        if (q < L.njobs && (int)blockIdx.x >= L.job[q].tile_begin) j = q;
    const int rows_wg = PAIR ? WR * 16 : SLOTS;
    const int row0 = ((int)blockIdx.x - L.job[j].tile_begin) * rows_wg;
    const int tok0 = (int)blockIdx.y * (WT * NT * 16) + wt * NT * 16;

    // which weight and row a slot s (= wr * MT * 16 + mt * 16 + rr) refers to
    auto slot_job = [&](int mt) { return PAIR ? mt : j; };
    auto slot_row = [&](int w_r, int mt, int rr) {
        return PAIR ? row0 + w_r * 16 + rr : row0 + w_r * MT * 16 + mt * 16 + rr;
    };

    // stage the block scales of the workgroup's rows: ps_lds[b * SLOTS + s]
    for (int idx = tid; idx < nb * SLOTS; idx += kGemmThreads) {
        const int b = idx / SLOTS, s = idx % SLOTS;
        const int w_r = s / (MT * 16), mt = (s / 16) % MT, rr = s % 16;
        const MvWeight& W = L.job[slot_job(mt)].W;
        const int r = min(slot_row(w_r, mt, rr), W.n - 1);
        ps_lds[idx] = W.ps[(size_t)r * nb + b];
    }

    // this lane's operand rows and token (clamped to valid memory; results outside are dropped)
    const uint8_t* arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const MvWeight& W = L.job[slot_job(mt)].W;
        const int r = min(slot_row(wr, mt, lane & 15), W.n - 1);
        arow[mt] = W.w + (size_t)r * nb * 64 + 16 * (lane >> 4);
    }
    const HyQ8K* brow[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) brow[n] = L.act + (size_t)min(tok0 + n * 16 + (lane & 15), nt - 1) * nb;
    int psh[MT], pof[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        psh[mt] = L.job[slot_job(mt)].W.pshift;
        pof[mt] = L.job[slot_job(mt)].W.poff;
    }

    auto load = [&](GemmFrag& f, int b) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) f.a[mt] = *reinterpret_cast<const uint4*>(arow[mt] + (size_t)b * 64);
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const HyQ8K* y = brow[n] + b;
#pragma unroll
            for (int l = 0; l < 4; l++) f.q[n][l] = *reinterpret_cast<const uint4*>(y->qp + 64 * l + 16 * (lane >> 4));
            const int2 ds = *reinterpret_cast<const int2*>(&y->d);
            f.d[n] = __builtin_bit_cast(float, ds.x);
            f.sum[n] = ds.y;
        }
    };

    float accf[MT][NT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 4; r++) accf[mt][n][r] = 0.f;

    GemmFrag cur, nxt;
    load(cur, 0);
    __syncthreads();  // ps_lds ready
    for (int b = 0; b < nb; b++) {
        load(nxt, min(b + 1, nb - 1));
        v4i acc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int n = 0; n < NT; n++) acc[mt][n] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int l = 0; l < 4; l++) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const v4i a = chunk_codes(cur.a[mt], l);
#pragma unroll
                for (int n = 0; n < NT; n++)
                    acc[mt][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, as_v4i(cur.q[n][l]), acc[mt][n], 0, 0, 0);
            }
        }
        // fp32 block terms, added in block order (src/kernels.c:576)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float4 ps4 =
                *reinterpret_cast<const float4*>(&ps_lds[b * SLOTS + wr * MT * 16 + mt * 16 + 4 * (lane >> 4)]);
            const float psr[4] = {ps4.x, ps4.y, ps4.z, ps4.w};
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float term =
                        psr[r] * cur.d[n] * (float)((acc[mt][n][r] << psh[mt]) - pof[mt] * cur.sum[n]);
                    accf[mt][n][r] = accf[mt][n][r] + term;
                }
        }
        cur = nxt;
    }

    // epilogue
    const int tl = lane & 15, rq = 4 * (lane >> 4);
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int t = tok0 + n * 16 + tl;
        if (t >= nt) continue;
        if (PAIR) {
            const GemmJob& J = L.job[0];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = slot_row(wr, 0, rq + r);
                if (row < J.W.n) {
                    const float g = accf[0][n][r], u = accf[1][n][r];
                    J.out[(size_t)t * J.ldo + row] = g / (1.0f + hy_expf(-g)) * u;
                }
            }
        } else {
            const GemmJob& J = L.job[j];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int row = slot_row(wr, mt, rq + r);
                    if (row < J.W.n) {
                        float* o = J.out + (size_t)t * J.ldo + row;
                        *o = J.epi == EPI_ADD ? *o + accf[mt][n][r] : accf[mt][n][r];
                    }
                }
        }
    }
}

template <int MT, int NT, int WR, int WT, bool PAIR>
hipError_t gemm_go(GemmLaunch& L, hipStream_t s) {
    const int rows_wg = PAIR ? WR * 16 : WR * MT * 16;
    int tiles = 0;
    for (int q = 0; q < L.njobs; q++) {
        L.job[q].tile_begin = tiles;
        if (!PAIR || q == 0) tiles += (L.job[q].W.n + rows_wg - 1) / rows_wg;
    }
    if (PAIR) L.job[1].tile_begin = 1 << 30;  // never selected by tile index
    const int toks_wg = WT * NT * 16;
    const dim3 grid(tiles, (L.nt + toks_wg - 1) / toks_wg);
    k_gemm_panel<MT, NT, WR, WT, PAIR><<<grid, kGemmThreads, 0, s>>>(L);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_panel(GemmLaunch& L, hipStream_t s) {
    if (L.njobs < 1 || L.njobs > kMaxJobs || L.nt < 1 || !L.act || (L.pair && L.njobs != 2)) return hipErrorInvalidValue;
    const int K = L.job[0].W.k;
    if (K % 256 || K / 256 > kGemmMaxNb) return hipErrorNotSupported;
    for (int q = 0; q < L.njobs; q++) {
        const MvWeight& W = L.job[q].W;
        if (W.kind != KIND_PANEL || W.k != K || W.nb != K / 256 || W.n < 1 || !L.job[q].out) return hipErrorNotSupported;
    }
    if (L.pair && L.job[0].W.n != L.job[1].W.n) return hipErrorNotSupported;
    L.nb = K / 256;
    if (L.pair) return gemm_go<2, 2, 2, 2, true>(L, s);
    return gemm_go<2, 2, 2, 2, false>(L, s);
}

}  // namespace hy
