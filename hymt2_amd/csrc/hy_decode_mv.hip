// Single-token matvec of the fused decode step (nt = 1), gfx950.
//
// Work layout: 256-thread workgroups, one weight row per half-wavefront per iteration, ITERS
// iterations per wave, so a workgroup covers 8 * ITERS rows (4 * ITERS gate/up pairs) and a
// launch has at most 192 workgroups where K = 2048 allows (256 for K = 6144). Lane j of a half-wavefront owns the 16-byte weight
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
#include "hy_mv_parts.h"

namespace hy {

namespace {

constexpr int kMv1Threads = 256;
constexpr int kMv1Waves = kMv1Threads / 64;
constexpr int kMv1MaxWgs = 256;

}  // namespace

// The fields of a job the kernel reads, for the weight kinds it may hold.
template <int KIND>
__device__ __forceinline__ void mv1_pin_job(const Mv1Job& J) {
    hy_sgpr_pin(J.W.w), hy_sgpr_pin(J.W.n), hy_sgpr_pin(J.out), hy_sgpr_pin(J.epi), hy_sgpr_pin(J.wg_begin);
    if (KIND == KIND_PANEL) hy_sgpr_pin(J.W.ps), hy_sgpr_pin(J.W.pshift), hy_sgpr_pin(J.W.poff);
    if (KIND == KIND_Q6K || KIND == KIND_ANY) hy_sgpr_pin(J.W.w2), hy_sgpr_pin(J.W.sc), hy_sgpr_pin(J.W.dh);
    if (KIND == KIND_ANY) hy_sgpr_pin(J.W.kind);
}

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
    // Every kernel argument this workgroup may use, loaded in one round of scalar loads and
    // pinned in SGPRs before any selection: selecting the job by its index first makes the
    // compiler load the chosen job's fields only once the index is known, several dependent
    // round trips to memory before the first vector load can issue.
    const Mv1Job j0 = L.job[0], j1 = L.job[1], j2 = L.job[2];
    const int pair = L.pair, njobs = L.njobs, rows_per_wg = L.rows_per_wg;
    const float* const lx = L.x;
    const float* const lnorm = L.norm_w;
    const HyQ8K* const lact = L.act;
    const float leps = L.eps;
    unsigned long long* const lslots = L.slots;
    const int n_arg = L.n_arg;
    hy_sgpr_pin(pair), hy_sgpr_pin(njobs), hy_sgpr_pin(rows_per_wg), hy_sgpr_pin(lx), hy_sgpr_pin(lnorm),
        hy_sgpr_pin(lact), hy_sgpr_pin(leps), hy_sgpr_pin(lslots), hy_sgpr_pin(n_arg);
    mv1_pin_job<KIND>(j0), mv1_pin_job<KIND>(j1), mv1_pin_job<KIND>(j2);
    int jsel = 0;
    if (!pair) {
        if (njobs > 1 && wg >= j1.wg_begin) jsel = 1;
        if (njobs > 2 && wg >= j2.wg_begin) jsel = 2;
    }
    const Mv1Job J = jsel == 0 ? j0 : (jsel == 1 ? j1 : j2);
    const bool up = pair && hh;  // pair mode: half-wave 1 streams the up rows
    const int kind = KIND == KIND_ANY ? J.W.kind : KIND;
    const uint8_t* w = up ? j1.W.w : J.W.w;
    const uint8_t* w2 = up ? j1.W.w2 : J.W.w2;
    const int8_t* wsc = up ? j1.W.sc : J.W.sc;
    const uint16_t* wdh = up ? j1.W.dh : J.W.dh;
    const float* wps = up ? j1.W.ps : J.W.ps;
    const int pshift = up ? j1.W.pshift : J.W.pshift;
    const int poff = up ? j1.W.poff : J.W.poff;
    const int n = J.W.n;
    const int row0 = (wg - J.wg_begin) * rows_per_wg;

    // 1. the prologue's inputs first (vector loads complete in issue order, so anything issued
    //    before the weights can be consumed without waiting for them); the residual of this
    //    lane's row as well. Wavefront w quantizes the blocks 2w*R .. 2w*R + 2R (R rounds of
    //    two blocks); a lane holds 8 consecutive elements of a block per round.
    constexpr int R = NB / (2 * kMv1Waves);
    float e[R][8], nw[R][8];
    float resid = 0.f;
    const int rrow = min(row0 + wave * RPW + lane, n - 1);  // the row this lane sums (lane < RPW)
    if (!pair && J.epi == EPI_ADD) resid = J.out[rrow];
    ActSeg A[SPL];
    if (PRO == PRO_NONE) {
#pragma unroll
        for (int s = 0; s < SPL; s++) A[s] = gather_act<SPB>(lact, kind, j + 32 * s);
    }
    if (PRO != PRO_NONE) {
#pragma unroll
        for (int k = 0; k < R; k++) {
            const int off = (2 * (wave * R + k)) * HY_QK + 8 * lane;
            const float4 v0 = *reinterpret_cast<const float4*>(lx + off);
            const float4 v1 = *reinterpret_cast<const float4*>(lx + off + 4);
            e[k][0] = v0.x, e[k][1] = v0.y, e[k][2] = v0.z, e[k][3] = v0.w;
            e[k][4] = v1.x, e[k][5] = v1.y, e[k][6] = v1.z, e[k][7] = v1.w;
            if (PRO == PRO_NORM) {
                const float4 u0 = *reinterpret_cast<const float4*>(lnorm + off);
                const float4 u1 = *reinterpret_cast<const float4*>(lnorm + off + 4);
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
        const int r = pair ? row0 + wave * ITERS + i : row0 + wave * RPW + 2 * i + hh;
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
            const float scale = 1.0f / sqrtf(sum / (float)K + leps);
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
            // every lane of the block holds the same term (its dot is reduced over the block's
            // lanes, its scales are the block's): an unconditional store, no exec-mask round trip
            terms[wave][rw][b] = t;
        }
    }
    __syncthreads();

    // 5. per-row sums in block order and the epilogue (optionally the greedy argmax of the rows,
    //    one key per workgroup)
    if (!pair) {
        unsigned long long key = 0ull;
        if (lane < RPW) {
            const int r = row0 + wave * RPW + lane;
            if (r < n) {
                float acc = 0.f;
#pragma unroll
                for (int b = 0; b < NB; b++) acc += terms[wave][lane][b];
                J.out[r] = J.epi == EPI_ADD ? resid + acc : acc;  // residual: h += tmp
                if (r < n_arg) key = argmax_key(acc, r);
            }
        }
        if (lslots) hy_wg_slot_max(key, lslots + wg);
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
        case 6: return mv1_pro<KIND, SPL, 6>(L, pro, grid, s);
        case 8: return mv1_pro<KIND, SPL, 8>(L, pro, grid, s);
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
    // the smallest ITERS whose grid is at most kMv1MaxWgs workgroups: every workgroup repeats
    // the prologue (load, RMSNorm, Q8_K), so fewer, longer workgroups measured faster, down to
    // 256 (the gate/up pairs: 256 against 192 workgroups +1.5 % decode; 384 and 512 lost 3-4 %)
    int iters = 0, grid = 0;
    const int max_iters = K == 2048 ? 8 : 1;
    for (int it = 1; it <= max_iters; it += it < 4 ? 1 : 2) {
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
    if (L.slots && (L.pair || grid > kArgSlots)) return hipErrorNotSupported;
    L.grid = grid;
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
