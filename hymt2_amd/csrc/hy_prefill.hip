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

// Workgroup barrier for LDS only: waits for this wave's LDS operations, not for its global
// loads, so prefetches stay in flight across it (a __syncthreads fence would drain them).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kTokRow = 272;  // LDS bytes per token row of qp: 256 + 16, so the 16 rows a
                              // B-fragment read touches start in 16 different bank groups

template <int MT, int NT, int WR, int WT, bool PAIR>
__global__ __launch_bounds__(kGemmThreads) void k_gemm_panel(GemmLaunch L) {
    static_assert(WR * WT == kGemmThreads / 64, "4 wavefronts per workgroup");
    static_assert(!PAIR || MT == 2, "pair mode: one gate and one up tile per wavefront");
    constexpr int SLOTS = WR * MT * 16;  // row slots of the workgroup
    constexpr int TOK = WT * NT * 16;    // tokens of the workgroup
    constexpr int BCH = TOK * 16 / kGemmThreads;  // 16-byte qp pieces per thread per block
    static_assert(BCH >= 1 && TOK <= kGemmThreads, "token tile");
    __shared__ __align__(16) float ps_lds[kGemmMaxNb * SLOTS];
    __shared__ __align__(16) uint8_t q_lds[2][TOK * kTokRow];
    __shared__ __align__(16) int2 ds_lds[2][TOK];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave % WR, wt = wave / WR;
    const int nb = L.nb, nt = L.nt;
    const HyQ8K* const act = L.act;

    // job of this row tile (uniform)
    int j = 0;
#pragma unroll
    for (int q = 1; q < kMaxJobs; q++)
        if (q < L.njobs && (int)blockIdx.x >= L.job[q].tile_begin) j = q;
    const int rows_wg = PAIR ? WR * 16 : SLOTS;
    const int row0 = ((int)blockIdx.x - L.job[j].tile_begin) * rows_wg;
    const int tokw = (int)blockIdx.y * TOK;  // first token of the workgroup

    auto slot_job = [&](int mt) { return PAIR ? mt : j; };
    auto slot_row = [&](int w_r, int mt, int rr) {
        return PAIR ? row0 + w_r * 16 + rr : row0 + w_r * MT * 16 + mt * 16 + rr;
    };

    // Per row tile: its weight (uniform; read from the kernel arguments with scalar loads: a
    // per-lane index into the job table would turn every field into a dependent vector load).
    const uint8_t* wbase[MT];
    const float* psbase[MT];
    int nrow[MT], psh[MT], pof[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const MvWeight& W = L.job[slot_job(mt)].W;
        wbase[mt] = W.w;
        psbase[mt] = W.ps;
        nrow[mt] = W.n;
        psh[mt] = W.pshift;
        pof[mt] = W.poff;
    }

    // Activations of one block for the workgroup's tokens: thread t loads 16-byte pieces
    // t, t + 256, ... of the TOK x 256 qp bytes (16 threads per token, coalesced), the first TOK
    // threads also (d, sum) of one token. Token indices are clamped to valid memory.
    v4i qreg[BCH];
    int2 dreg = make_int2(0, 0);
    const int8_t* qsrc[BCH];
#pragma unroll
    for (int i = 0; i < BCH; i++) {
        const int q = tid + i * kGemmThreads;
        qsrc[i] = act[(size_t)min(tokw + (q >> 4), nt - 1) * nb].qp + 16 * (q & 15);
    }
    const int2* dsrc = reinterpret_cast<const int2*>(&act[(size_t)min(tokw + (tid % TOK), nt - 1) * nb].d);
    auto qload = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < BCH; i++)
            qreg[i] = *reinterpret_cast<const v4i*>(qsrc[i] + (size_t)b * sizeof(HyQ8K));
        if (tid < TOK) dreg = *reinterpret_cast<const int2*>(reinterpret_cast<const char*>(dsrc) + (size_t)b * sizeof(HyQ8K));
    };
    auto qstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            const int q = tid + i * kGemmThreads;
            *reinterpret_cast<v4i*>(&q_lds[buf][(q >> 4) * kTokRow + 16 * (q & 15)]) = qreg[i];
        }
        if (tid < TOK) ds_lds[buf][tid] = dreg;
    };

    // this lane's weight rows (clamped; results outside are dropped)
    const uint8_t* arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int r = min(slot_row(wr, mt, lane & 15), nrow[mt] - 1);
        arow[mt] = wbase[mt] + (size_t)r * nb * 64 + 16 * (lane >> 4);
    }
    uint4 a0[MT], a1[MT];
    auto aload = [&](uint4 (&a)[MT], int b) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) a[mt] = *reinterpret_cast<const uint4*>(arow[mt] + (size_t)b * 64);
    };

    // first block's operands, then the block scales of the workgroup's rows: ps_lds[b][slot]
    qload(0);
    aload(a0, 0);
    {
        constexpr int ROWS = WR * 16;                          // rows of one row-tile slice
        constexpr int CNT = kGemmMaxNb * ROWS / kGemmThreads;  // entries per thread per slice
        float v[MT][CNT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < CNT; i++) {
                const int idx = tid + i * kGemmThreads;
                const int b = min(idx / ROWS, nb - 1), q = idx % ROWS;
                const int r = min(slot_row(q / 16, mt, q % 16), nrow[mt] - 1);
                v[mt][i] = psbase[mt][(size_t)r * nb + b];
            }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < CNT; i++) {
                const int idx = tid + i * kGemmThreads;
                const int b = idx / ROWS, q = idx % ROWS;
                if (b < nb) ps_lds[b * SLOTS + (q / 16) * MT * 16 + mt * 16 + q % 16] = v[mt][i];
            }
    }
    qstore(0);

    float accf[MT][NT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 4; r++) accf[mt][n][r] = 0.f;

    const int tl = lane & 15, g = lane >> 4;
    // one block: MFMAs over its four K = 64 chunks, then the fp32 terms added in block order
    // (src/kernels.c:576: ps * d * (float)((enc << pshift) - poff * sum))
    auto compute = [&](const uint4 (&a)[MT], int b, int buf) __attribute__((always_inline)) {
        v4i acc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int n = 0; n < NT; n++) acc[mt][n] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int l = 0; l < 4; l++) {
            uint4 qv[NT];
#pragma unroll
            for (int n = 0; n < NT; n++)
                qv[n] = *reinterpret_cast<const uint4*>(
                    &q_lds[buf][(wt * NT * 16 + n * 16 + tl) * kTokRow + 64 * l + 16 * g]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const v4i av = chunk_codes(a[mt], l);
#pragma unroll
                for (int n = 0; n < NT; n++)
                    acc[mt][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, as_v4i(qv[n]), acc[mt][n], 0, 0, 0);
            }
        }
        float dn[NT];
        int off[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int2 ds = ds_lds[buf][wt * NT * 16 + n * 16 + tl];
            dn[n] = __builtin_bit_cast(float, ds.x);
            off[n] = ds.y;
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float4 ps4 = *reinterpret_cast<const float4*>(&ps_lds[b * SLOTS + wr * MT * 16 + mt * 16 + 4 * g]);
            const float psr[4] = {ps4.x, ps4.y, ps4.z, ps4.w};
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const int sub = pof[mt] * off[n];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float term = psr[r] * dn[n] * (float)((acc[mt][n][r] << psh[mt]) - sub);
                    accf[mt][n][r] = accf[mt][n][r] + term;
                }
            }
        }
    };

    lds_barrier();  // ps_lds and block 0 in LDS
    for (int b = 0; b < nb; b += 2) {
        // block b from buffer 0 with a0; block b + 1 loaded meanwhile (clamped, unused past the end)
        const int b1 = min(b + 1, nb - 1);
        qload(b1);
        aload(a1, b1);
        compute(a0, b, 0);
        __builtin_amdgcn_sched_barrier(0);  // the LDS stores wait for the loads: after the terms
        qstore(1);
        lds_barrier();
        if (b + 1 >= nb) break;
        const int b2 = min(b + 2, nb - 1);
        qload(b2);
        aload(a0, b2);
        compute(a1, b + 1, 1);
        __builtin_amdgcn_sched_barrier(0);
        qstore(0);
        lds_barrier();
    }

    // epilogue: lane holds rows 4 g .. 4 g + 3 of each row tile for token tl of each token tile
    float* const out = L.job[j].out;
    const int ldo = L.job[j].ldo, nout = L.job[j].W.n, epi = L.job[j].epi;
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int t = tokw + wt * NT * 16 + n * 16 + tl;
        if (t >= nt) continue;
        if (PAIR) {
            const int row = slot_row(wr, 0, 4 * g);
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float gt = accf[0][n][r], up = accf[1][n][r];
                v[r] = gt / (1.0f + hy_expf(-gt)) * up;
            }
            float* o = out + (size_t)t * ldo + row;
            if (row + 3 < nout && ((ldo | row) & 3) == 0) {
                *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                    if (row + r < nout) o[r] = v[r];
            }
        } else {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int row = slot_row(wr, mt, 4 * g);
                float* o = out + (size_t)t * ldo + row;
                if (row + 3 < nout && ((ldo | row) & 3) == 0) {
                    float4 v = make_float4(accf[mt][n][0], accf[mt][n][1], accf[mt][n][2], accf[mt][n][3]);
                    if (epi == EPI_ADD) {
                        const float4 h = *reinterpret_cast<const float4*>(o);
                        v = make_float4(h.x + v.x, h.y + v.y, h.z + v.z, h.w + v.w);
                    }
                    *reinterpret_cast<float4*>(o) = v;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (row + r < nout) o[r] = epi == EPI_ADD ? o[r] + accf[mt][n][r] : accf[mt][n][r];
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
