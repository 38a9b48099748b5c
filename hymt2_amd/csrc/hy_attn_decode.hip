// Single-token attention of the fused decode step (nt = 1), gfx950: one 256-thread workgroup
// per query head, the reference's attn_task for one position (src/model.c:767-795) after the
// per-token RoPE, q/k RMSNorm and bf16 KV store (src/model.c:836-847).
//
// Latency plan: the key rows of the first 256 positions and the value tile of the first 128
// positions are loaded at kernel entry, so their HBM latency overlaps the RoPE + RMSNorm of
// this token. Scores: one key per thread, dot_bf16's four interleaved partial sums in order
// (src/kernels.c:1111-1121). Softmax: max (order-free), expf, the sum in position order, the
// probabilities p_j = e_j * (1 / sum). Output: one lane per head dimension accumulates
// o += p_j * V_j[d] in position order (axpy_bf16, src/kernels.c:1122-1124) from LDS tiles of
// 128 positions; the next tile is loaded while the current one is summed. The fp32 output row
// goes to `ao`; the o-projection quantizes it.
#include "hy_kernels.h"

namespace hy {

namespace {

constexpr int kA1Threads = 256;
constexpr int kA1Keys = 256;  // keys per score pass (one per thread)
constexpr int kA1Tile = 128;  // positions per V tile in LDS

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
#pragma unroll
    for (int i = 0; i < RPL; i++) scr[lane + 64 * i] = x[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float r[RPL];
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

template <int HD>
__global__ __launch_bounds__(kA1Threads) void k_attn1(Attn1Args a) {
    constexpr int KV4 = HD / 8;                           // 16-byte pieces of one K / V row
    constexpr int RPL = HD / 64;                          // row elements per lane
    constexpr int VT_LOADS = kA1Tile * KV4 / kA1Threads;  // V pieces per thread per tile
    static_assert(VT_LOADS >= 1 && kA1Tile * KV4 % kA1Threads == 0, "tile split");
    __shared__ __align__(16) uint16_t vt[kA1Tile * HD];   // V tile, natural layout vt[j][d]
    __shared__ __align__(16) float scr[2][HD];
    __shared__ __align__(16) float qn[HD];
    __shared__ __align__(16) uint16_t kb[HD];
    __shared__ __align__(16) uint16_t vb[HD];
    __shared__ float red[kA1Threads / 64];
    __shared__ float stat;
    extern __shared__ __align__(16) float ex[];           // scores, exponentials, probabilities [n]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x;
    const int group = a.heads / a.kv_heads;
    const int g = h / group;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos0;
    const int n = pos + 1;
    const int half = a.rope_half;
    const uint16_t* K = a.kc + (size_t)g * a.ctx * HD;
    const uint16_t* V = a.vc + (size_t)g * a.ctx * HD;

    // 0. loads: this token's row (wavefronts 0: q, 1: k, 2: v) with its RoPE table entries and
    //    norm weights, then the cached K rows of the first pass (one key per thread)
    float x[RPL], rc[RPL], rs[RPL], nw[RPL];
    {
        const float* src = wave == 0 ? a.q + (size_t)h * HD : (wave == 1 ? a.k + (size_t)g * HD : a.v + (size_t)g * HD);
        const float* nsrc = wave == 0 ? a.q_norm : a.k_norm;
        const float* cs = a.rope_cos + (size_t)pos * half;
        const float* sn = a.rope_sin + (size_t)pos * half;
#pragma unroll
        for (int i = 0; i < RPL; i++) {
            const int d = lane + 64 * i, t = d < half ? d : (d < 2 * half ? d - half : 0);
            x[i] = src[d];
            rc[i] = cs[t];
            rs[i] = sn[t];
            nw[i] = nsrc[d];
        }
    }
    uint4 kr[KV4];
    if (tid < pos) {
#pragma unroll
        for (int i = 0; i < KV4; i++) kr[i] = *reinterpret_cast<const uint4*>(K + (size_t)tid * HD + 8 * i);
    }
    a1_fence();

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
    // the first V tile's loads (natural layout: consecutive threads, consecutive pieces of a row)
    uint4 vr[VT_LOADS];
#pragma unroll
    for (int i = 0; i < VT_LOADS; i++) {
        const int f = tid + kA1Threads * i, j = f / KV4;
        if (j < pos) vr[i] = *reinterpret_cast<const uint4*>(V + (size_t)j * HD + 8 * (f % KV4));
    }
    __syncthreads();
    // the bf16 k, v of this position (src/model.c:842-847), stored once per KV head
    if (h % group == 0 && tid < HD) {
        const size_t off = ((size_t)g * a.ctx + pos) * HD + tid;
        a.kc[off] = kb[tid];
        a.vc[off] = vb[tid];
    }

    // 2. scores s_j = dot_bf16(q, K_j) * (1/sqrtf(hd)); key `pos` is this token's kb
    const float scale = 1.0f / sqrtf((float)HD);
    float lmax = -__builtin_inff();
    for (int p0 = 0; p0 < n; p0 += kA1Keys) {
        const int j = p0 + tid;
        if (p0 > 0 && j < pos) {
#pragma unroll
            for (int i = 0; i < KV4; i++) kr[i] = *reinterpret_cast<const uint4*>(K + (size_t)j * HD + 8 * i);
        }
        if (j < n) {
            float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
            for (int i = 0; i < KV4; i++) {
                float kf[8];
                bf16x8f(j == pos ? *reinterpret_cast<const uint4*>(kb + 8 * i) : kr[i], kf);
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
            const float sj = ((a0 + a1) + (a2 + a3)) * scale;
            ex[j] = sj;
            lmax = fmaxf(lmax, sj);
        }
    }
    lmax = hy_wave_max(lmax);
    if (lane == 0) red[wave] = lmax;

    // 3. softmax over positions (src/model.c:781-789): max (order-free), exp, sum in order,
    //    p_j = e_j * (1 / sum); the first V tile goes into LDS meanwhile
    auto store_tile = [&](int t0) {
#pragma unroll
        for (int i = 0; i < VT_LOADS; i++) {
            const int f = tid + kA1Threads * i, jj = f / KV4, pc = f % KV4;
            const uint4 val = t0 + jj == pos ? *reinterpret_cast<const uint4*>(vb + 8 * pc) : vr[i];
            *reinterpret_cast<uint4*>(vt + (size_t)jj * HD + 8 * pc) = val;
        }
    };
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int j = tid; j < n; j += kA1Threads) ex[j] = hy_expf(ex[j] - mx);
    store_tile(0);
    __syncthreads();
    if (wave == 0) {
        const float sum = hy_wave_seq_sum(ex, n, lane);
        if (lane == 0) stat = 1.0f / sum;
    }
    __syncthreads();
    const float inv = stat;
    for (int j = tid; j < n; j += kA1Threads) ex[j] = ex[j] * inv;  // sc[j] * inv, once per position
    __syncthreads();

    // 4. o[d] = sum_j p_j * V_j[d] in position order (axpy_bf16), one lane per dimension
    float o = 0.f;
    for (int t0 = 0; t0 < n; t0 += kA1Tile) {
        if (t0 > 0) {
            __syncthreads();  // previous tile consumed
            store_tile(t0);
            __syncthreads();
        }
        if (t0 + kA1Tile < n) {  // the next tile's loads, in flight while this one is summed
#pragma unroll
            for (int i = 0; i < VT_LOADS; i++) {
                const int f = tid + kA1Threads * i, j = t0 + kA1Tile + f / KV4;
                if (j < pos) vr[i] = *reinterpret_cast<const uint4*>(V + (size_t)j * HD + 8 * (f % KV4));
            }
        }
        if (tid < HD) {
            const int cnt = min(kA1Tile, n - t0);
            const float* pj = ex + t0;
            const uint16_t* vd = vt + tid;
            int jj = 0;
            for (; jj + 8 <= cnt; jj += 8) {
                const float4 p0 = *reinterpret_cast<const float4*>(pj + jj);
                const float4 p1 = *reinterpret_cast<const float4*>(pj + jj + 4);
                const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
                float vv[8];
#pragma unroll
                for (int k = 0; k < 8; k++) vv[k] = hy_bf16(vd[(size_t)(jj + k) * HD]);
#pragma unroll
                for (int k = 0; k < 8; k++) o += pv[k] * vv[k];
            }
            for (; jj < cnt; jj++) o += pj[jj] * hy_bf16(vd[(size_t)jj * HD]);
        }
    }
    if (tid < HD) a.ao[(size_t)h * HD + tid] = o;
}

size_t attn1_lds(int ctx) { return ((size_t)ctx + 8) * sizeof(float); }

hipError_t launch_attn1(const Attn1Args& a, hipStream_t s) {
    if (a.heads % a.kv_heads || 2 * a.rope_half > a.hdim || a.ctx > kA1MaxCtx) return hipErrorNotSupported;
    const size_t lds = attn1_lds(a.ctx);
    switch (a.hdim) {
    case 64: k_attn1<64><<<a.heads, kA1Threads, lds, s>>>(a); break;
    case 128: k_attn1<128><<<a.heads, kA1Threads, lds, s>>>(a); break;
    default: return hipErrorNotSupported;
    }
    return hipGetLastError();
}

}  // namespace hy
