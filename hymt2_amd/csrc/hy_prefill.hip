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
// (src/model.c:873-876) has both values in one register. Each K-block's operands (activation
// pieces, panel bytes, token scales and sums, row block scales) land in a stage of an LDS ring
// by direct global -> LDS loads, the next blocks' in flight while the current block's MFMAs
// run.
#include <algorithm>

#include "hy_kernels.h"

namespace hy {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;

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

// Direct global -> LDS loads: lane L's 16 (4) bytes from src land at LDS address dst + 16 L
// (4 L), dst uniform (an LDS byte address). Written as assembly so that the compiler does not
// order the workgroup's LDS reads behind them: the kernel waits for them itself (wait_vm), for
// the block it is about to read, and the LDS they fill is not read before that wait.
// An LDS-DMA load that reads M0 right after a scalar write of M0 needs one wait state on this
// family (the compiler's hazard pass does not look inside the assembly): the s_nop provides it;
// without it the load may take the previous M0 and fill another piece's slot.
__device__ __forceinline__ void dma16(const void* src, uint32_t dst) {
    const uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* src, uint32_t dst) {
    const uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// Waits until at most N of this wave's vector memory operations (loads, LDS-direct loads) are
// outstanding. They complete in issue order.
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One K-block of operands in LDS, filled by direct loads (no registers):
//   q: the workgroup's TOK tokens x 16 pieces of 16 qp bytes; piece c of token t sits at slot
//      16 t + (c ^ (t & 15)), so the 16 tokens of a B-fragment read hit 16 bank groups;
//   a: the workgroup's ROWS panel rows x 4 pieces of 16 bytes; piece g of row r at slot
//      4 r + (g ^ ((r >> 2) & 3)), conflict-free the same way for the A-fragment reads;
//   d, sum: the tokens' Q8_K scale and sum (one 64-lane direct load each); ps: the rows' block
//   scales (one 64-lane direct load per 64 row slots).
template <int ROWS, int TOK>
struct GemmStage {
    alignas(16) uint8_t q[TOK * 256];
    alignas(16) uint8_t a[ROWS * 64];
    alignas(16) float d[64];
    alignas(16) int sum[64];
    alignas(16) float ps[ROWS > 64 ? 128 : 64];
};

// KS = 2 splits K inside the workgroup: two sets of 4 wavefronts own the same output tile,
// set 0 the first NBH blocks, set 1 the last NBH, stepping together through one barrier per
// block pair. Set 0 keeps the running sum in block order; set 1 keeps its NBH fp32 block terms
// in registers and, after set 0 hands its sums over through LDS, adds them in block order, so
// each output is the same sequential sum as with KS = 1.
template <int NJ, int MT, int NT, int WR, int WT, bool PAIR, int RING, int KS = 1, int NBH = 0>
__global__ __launch_bounds__(kGemmThreads * KS) void k_gemm_panel(GemmLaunchT<NJ> L) {
    static_assert(WR * WT == kGemmThreads / 64, "4 wavefronts per workgroup (per K set)");
    static_assert(KS == 1 || (KS == 2 && NBH >= 1), "K split in two halves of NBH blocks");
    static_assert(!PAIR || MT == 2, "pair mode: one gate and one up tile per wavefront");
    constexpr int SLOTS = WR * MT * 16;  // row slots of the workgroup
    constexpr int TOK = WT * NT * 16;    // tokens of the workgroup
    // direct loads of one block: QN of qp, AN of panel bytes, then d, sum and the rows' block
    // scales (64 lanes each), dealt round-robin to the wavefronts: load k goes to wavefront k % 4
    constexpr int QN = TOK / 4, AN = SLOTS / 16, PSN = (SLOTS + 63) / 64, TOTAL = QN + AN + 2 + PSN;
    constexpr int MAXI = (TOTAL + 3) / 4;
    static_assert(TOK % 4 == 0 && SLOTS % 16 == 0 && TOK <= 64, "tile shape");
    static_assert(SLOTS <= 128, "the row block scales are at most two 64-lane loads per block");
    using Stage = GemmStage<SLOTS, TOK>;
    __shared__ Stage ring[RING * KS];
    __shared__ __align__(16) float xch[KS == 2 ? kGemmThreads * MT * NT * 4 : 4];  // set 0's sums
    __shared__ uint64_t etab[PAIR ? 32 : 1];  // expf table of the SwiGLU epilogue (LDS lookups)

    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3;
    if (PAIR && tid < 32) etab[tid] = hy_exp_tab_entry(tid);  // read after the block barriers
    const int half = KS == 2 ? __builtin_amdgcn_readfirstlane(tid >> 8) : 0;  // K set
    const int wr = wave % WR, wt = wave / WR;
    const int nb = L.nb;
    const int nbh = KS == 2 ? NBH : nb;  // blocks of this K set, from block hb0
    const int hb0 = half * nbh;

    // job of this row tile (uniform; in pair mode only the gate jobs 2p carry tiles)
    int j = 0;
#pragma unroll
    for (int q = 1; q < NJ; q++)
        if (q < L.njobs && (int)blockIdx.x >= L.job[q].tile_begin) j = q;
    const int rows_wg = PAIR ? WR * 16 : SLOTS;
    const int row0 = ((int)blockIdx.x - L.job[j].tile_begin) * rows_wg;
    const int tokw = (int)blockIdx.y * TOK;  // first token of the workgroup
    const HyQ8K* const act = L.job[j].act;  // a pair's gate and up share their tokens
    const int nt = L.job[j].nt;
    if (tokw >= nt) return;  // a shorter chunk of a pipelined launch (uniform)

    auto slot_job = [&](int mt) { return PAIR ? j + mt : j; };
    // weight row of local row slot s = w_r * MT * 16 + mt * 16 + rr
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

    // Sources of this thread's direct loads for block 0 (block b adds b times the stride) and
    // their LDS destinations (offsets in a stage)
    const char* src[MAXI];
    size_t stride[MAXI];
    uint32_t dst[MAXI];
#pragma unroll
    for (int i = 0; i < MAXI; i++) {
        const int k = min(wave + 4 * i, TOTAL - 1);
        if (k < QN) {
            const int sl = k * 64 + lane, t = sl >> 4, c = (sl & 15) ^ (t & 15);
            src[i] = reinterpret_cast<const char*>(act[(size_t)min(tokw + t, nt - 1) * nb].qp + 16 * c);
            stride[i] = sizeof(HyQ8K);
            dst[i] = offsetof(Stage, q) + k * 1024;
        } else if (k < QN + AN) {
            const int sl = (k - QN) * 64 + lane, r = sl >> 2, gg = (sl & 3) ^ ((r >> 2) & 3);
            const int w_r = r / (MT * 16), mt = (r / 16) % MT, rr = r % 16;
            // mt is per lane here: select among the row tiles' bases with constant indices
            const uint8_t* wb = wbase[0];
            int nr = nrow[0];
#pragma unroll
            for (int m = 1; m < MT; m++)
                if (mt == m) wb = wbase[m], nr = nrow[m];
            src[i] = reinterpret_cast<const char*>(wb + (size_t)min(slot_row(w_r, mt, rr), nr - 1) * nb * 64 + 16 * gg);
            stride[i] = 64;
            dst[i] = offsetof(Stage, a) + (k - QN) * 1024;
        } else if (k < QN + AN + 2) {
            src[i] = reinterpret_cast<const char*>(&act[(size_t)min(tokw + lane, nt - 1) * nb].d) + (k == QN + AN ? 0 : 4);
            stride[i] = sizeof(HyQ8K);
            dst[i] = k == QN + AN ? offsetof(Stage, d) : offsetof(Stage, sum);
        } else {  // block scale of row slot 64 part + lane (slots past SLOTS load a valid row, unused)
            const int part = k - (QN + AN + 2);
            const int sl = min(64 * part + lane, SLOTS - 1);
            const int w_r = sl / (MT * 16), mt = (sl / 16) % MT, rr = sl % 16;
            const float* pb = psbase[0];
            int nr = nrow[0];
#pragma unroll
            for (int m = 1; m < MT; m++)
                if (mt == m) pb = psbase[m], nr = nrow[m];
            src[i] = reinterpret_cast<const char*>(pb + (size_t)min(slot_row(w_r, mt, rr), nr - 1) * nb);
            stride[i] = 4;
            dst[i] = offsetof(Stage, ps) + 256 * part;
        }
    }
    const uint32_t ring0 = lds_addr(&ring[0]);
    // block hb0 + b of this K set into ring slot buf
    auto issue = [&](int b, int buf) __attribute__((always_inline)) {
        const uint32_t base = ring0 + (buf * KS + half) * (uint32_t)sizeof(Stage);
#pragma unroll
        for (int i = 0; i < MAXI; i++) {
            const int k = wave + 4 * i;
            if (k < QN + AN) dma16(src[i] + (size_t)(hb0 + b) * stride[i], base + dst[i]);
            else if (k < TOTAL) dma4(src[i] + (size_t)(hb0 + b) * stride[i], base + dst[i]);
        }
    };

    // the first RING - 1 blocks (clamped: a block past the end repeats the last, unused)
#pragma unroll
    for (int b = 0; b < RING - 1; b++) issue(min(b, nbh - 1), b);

    float accf[MT][NT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 4; r++) accf[mt][n][r] = 0.f;

    const int tl = lane & 15, g = lane >> 4;
    // one block step: the fp32 terms of block hb0 + b for this wavefront's outputs
    auto step = [&](int b, float (&term)[MT][NT][4]) __attribute__((always_inline)) {
        const int buf = b % RING;
        // block b's direct loads are the oldest RING - 1 issues ago: wait for them, then the
        // barrier makes every wavefront's share visible (and ends the reads of block b - 1,
        // whose buffer the next issue refills)
        // this wavefront's loads per block: the k < TOTAL with k % 4 == wave
        if (wave == 0) wait_vm<(RING - 2) * ((TOTAL + 3) / 4)>();
        else if (wave == 1) wait_vm<(RING - 2) * ((TOTAL + 2) / 4)>();
        else if (wave == 2) wait_vm<(RING - 2) * ((TOTAL + 1) / 4)>();
        else wait_vm<(RING - 2) * (TOTAL / 4)>();
        hy_lds_barrier();
        issue(min(b + RING - 1, nbh - 1), (b + RING - 1) % RING);
        const Stage& S = ring[buf * KS + half];

        // MFMAs over the block's four K = 64 chunks
        v4i acc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int n = 0; n < NT; n++) acc[mt][n] = v4i{0, 0, 0, 0};
        uint4 ap[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int r = wr * MT * 16 + mt * 16 + tl;
            ap[mt] = *reinterpret_cast<const uint4*>(S.a + (4 * r + (g ^ ((r >> 2) & 3))) * 16);
        }
#pragma unroll
        for (int l = 0; l < 4; l++) {
            v4i qv[NT];
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const int t = wt * NT * 16 + n * 16 + tl;
                qv[n] = *reinterpret_cast<const v4i*>(S.q + (16 * t + ((4 * l + g) ^ tl)) * 16);
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const v4i av = chunk_codes(ap[mt], l);
#pragma unroll
                for (int n = 0; n < NT; n++)
                    acc[mt][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, qv[n], acc[mt][n], 0, 0, 0);
            }
        }
        // fp32 terms added in block order (src/kernels.c:576: ps * d * (float)((enc << pshift)
        // - poff * sum))
        float dn[NT];
        int off[NT];
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const int t = wt * NT * 16 + n * 16 + tl;
            dn[n] = S.d[t];
            off[n] = S.sum[t];
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float4 ps4 = *reinterpret_cast<const float4*>(&S.ps[wr * MT * 16 + mt * 16 + 4 * g]);
            const float psr[4] = {ps4.x, ps4.y, ps4.z, ps4.w};
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const int nsub = -(pof[mt] * off[n]);
#pragma unroll
                for (int r = 0; r < 4; r++) term[mt][n][r] = psr[r] * dn[n] * (float)((acc[mt][n][r] << psh[mt]) + nsub);
            }
        }
    };
    auto accumulate = [&](const float (&term)[MT][NT][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int r = 0; r < 4; r++) accf[mt][n][r] = accf[mt][n][r] + term[mt][n][r];
    };
    if constexpr (KS == 1) {
        for (int b = 0; b < nb; b++) {
            float term[MT][NT][4];
            step(b, term);
            accumulate(term);
        }
        wait_vm<0>();  // the clamped trailing issues complete before the workgroup ends
    } else {
        float tm[NBH][MT][NT][4];
#pragma unroll
        for (int b = 0; b < NBH; b++) {
            step(b, tm[b]);
            if (half == 0) accumulate(tm[b]);
        }
        wait_vm<0>();
        // set 0 hands its sums over; set 1 adds its terms after them, in block order, and stores
        float4* xv = reinterpret_cast<float4*>(xch) + (size_t)(wave * 64 + lane) * (MT * NT);
        if (half == 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int n = 0; n < NT; n++)
                    xv[mt * NT + n] = make_float4(accf[mt][n][0], accf[mt][n][1], accf[mt][n][2], accf[mt][n][3]);
        }
        __syncthreads();
        if (half == 0) return;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const float4 p = xv[mt * NT + n];
                accf[mt][n][0] = p.x, accf[mt][n][1] = p.y, accf[mt][n][2] = p.z, accf[mt][n][3] = p.w;
            }
#pragma unroll
        for (int b = 0; b < NBH; b++) accumulate(tm[b]);
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
                v[r] = gt / (1.0f + hy_expf_tab(-gt, etab)) * up;
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

template <int NJ, int MT, int NT, int WR, int WT, bool PAIR, int RING, int KS = 1, int NBH = 0>
hipError_t gemm_go(GemmLaunchT<NJ>& L, hipStream_t s) {
    const int rows_wg = PAIR ? WR * 16 : WR * MT * 16;
    int tiles = 0;
    for (int q = 0; q < L.njobs; q++) {
        if (PAIR && q % 2) {
            L.job[q].tile_begin = 1 << 30;  // an up job: never selected by tile index
            continue;
        }
        L.job[q].tile_begin = tiles;
        tiles += (L.job[q].W.n + rows_wg - 1) / rows_wg;
    }
    const int toks_wg = WT * NT * 16;
    const dim3 grid(tiles, (L.nt + toks_wg - 1) / toks_wg);
    k_gemm_panel<NJ, MT, NT, WR, WT, PAIR, RING, KS, NBH><<<grid, kGemmThreads * KS, 0, s>>>(L);
    return hipGetLastError();
}

// Checks the jobs and completes the launch: per-job activations default to the launch's, L.nt
// becomes the largest job's token count. A launch holds one K; in pair mode jobs (2p, 2p + 1)
// are the gate and up weights of equal rows over the same tokens.
template <int NJ>
hipError_t gemm_prepare(GemmLaunchT<NJ>& L) {
    if (L.njobs < 1 || L.njobs > NJ || (L.pair && L.njobs % 2)) return hipErrorInvalidValue;
    const int K = L.job[0].W.k;
    if (K % 256) return hipErrorNotSupported;
    int ntmax = 0;
    for (int q = 0; q < L.njobs; q++) {
        GemmJob& J = L.job[q];
        const MvWeight& W = J.W;
        if (W.kind != KIND_PANEL || W.k != K || W.nb != K / 256 || W.n < 1 || !J.out) return hipErrorNotSupported;
        if (!J.act) {
            J.act = L.act;
            J.nt = L.nt;
        }
        if (!J.act || J.nt < 1) return hipErrorInvalidValue;
        if (L.pair && q % 2 && (W.n != L.job[q - 1].W.n || J.act != L.job[q - 1].act || J.nt != L.job[q - 1].nt))
            return hipErrorNotSupported;
        ntmax = std::max(ntmax, J.nt);
    }
    L.nt = ntmax;
    L.nb = K / 256;
    return hipSuccess;
}

template <int NJ>
hipError_t gemm_dispatch(GemmLaunchT<NJ>& L, hipStream_t s) {
    const hipError_t e = gemm_prepare(L);
    if (e != hipSuccess) return e;
    // tiles and ring depths as measured fastest in chunked prefill (128 tokens): gate/up pairs in
    // 32-token tiles with two ring stages, the other contractions in the largest tile that still
    // gives a workgroup per CU (else the smallest) with three
    int rows = 0;
    for (int q = 0; q < L.njobs; q++)
        if (!L.pair || q % 2 == 0) rows += L.job[q].W.n;
    auto wgs = [&](int rt, int tt) { return ((rows + rt - 1) / rt) * ((L.nt + tt - 1) / tt); };
    // K = 2048 and 6144 (8 and 24 blocks) outside pair mode: K split in two inside the
    // workgroup (measured slower for the gate/up pairs)
    // pipelined launches (up to 8 chunks of 128 tokens): 64-token tiles and two ring stages
    // throughout, as measured fastest on eight stacked jobs of each shape (gate/up 88.5 ->
    // 71.2 us, qkv 25.5 -> 20.9 us); gate/up pairs in 64 pairs x 64 tokens with the four
    // wavefronts down the rows when that still gives a workgroup per CU (eight stacked jobs:
    // 71-75 -> 57 us; 128-row tiles of the other shapes measured within noise)
    if constexpr (NJ == kGemmPipeJobs) {
        if (L.pair) return wgs(64, 64) >= 256 ? gemm_go<NJ, 2, 4, 4, 1, true, 2>(L, s) : gemm_go<NJ, 2, 2, 2, 2, true, 2>(L, s);
        if (wgs(64, 64) >= 256) return gemm_go<NJ, 2, 2, 2, 2, false, 2>(L, s);
    }
    if (L.pair) return gemm_go<NJ, 2, 1, 2, 2, true, 2>(L, s);
    // large single contractions (8192+ rows at 128 tokens; none in a layer of the 1.8B model):
    // 64 rows x 32 tokens, the four wavefronts down the rows, two ring stages (the 12288 x 2048
    // panel over 128 tokens: 12.1 against 15.2 us with 64 x 64 tiles and three stages)
    if (wgs(64, 64) >= 256) return gemm_go<NJ, 1, 2, 4, 1, false, 2>(L, s);
    // K = 2048, one chunk (qkv: 3072 rows, o: 2048): the four wavefronts of each K set down the
    // rows, two ring stages (qkv 8.2 -> 6.7 us with 32-token tiles, o 6.3 -> 5.9 us with 16)
    if (L.nb == 8) return rows >= 3072 ? gemm_go<NJ, 1, 2, 4, 1, false, 2, 2, 4>(L, s) : gemm_go<NJ, 1, 1, 4, 1, false, 2, 2, 4>(L, s);
    if (L.nb == 24) return gemm_go<NJ, 1, 1, 2, 2, false, 3, 2, 12>(L, s);
    return gemm_go<NJ, 1, 1, 2, 2, false, 3>(L, s);
}

}  // namespace

hipError_t launch_gemm_panel(GemmLaunch& L, hipStream_t s) { return gemm_dispatch(L, s); }
hipError_t launch_gemm_panel(GemmPipeLaunch& L, hipStream_t s) { return gemm_dispatch(L, s); }

}  // namespace hy
