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

template <int HD>
__global__ __launch_bounds__(kA1Threads) void k_attn1(Attn1Args a) {
    constexpr int KV4 = HD / 8;                              // 16-byte pieces of one K / V row
    constexpr int VT_LOADS = kA1Tile * KV4 / kA1Threads;     // 16-byte V loads per thread per tile
    static_assert(VT_LOADS >= 1 && kA1Tile * KV4 % kA1Threads == 0, "tile split");
    __shared__ __align__(16) uint16_t vt[kA1Tile * HD];
    __shared__ __align__(16) float row[3][HD];  // q, k, v of this token
    __shared__ __align__(16) uint16_t kb[HD];
    __shared__ __align__(16) uint16_t vb[HD];
    __shared__ float red[kA1Threads / 64];
    __shared__ float stat[2];
    extern __shared__ __align__(16) float sc[];  // scores, then probabilities [n]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x;
    const int group = a.heads / a.kv_heads;
    const int g = h / group;
    const int pos = a.pos_dev ? *a.pos_dev : a.pos0;
    const int n = pos + 1;
    const int half = a.rope_half;
    const uint16_t* K = a.kc + (size_t)g * a.ctx * HD;
    const uint16_t* V = a.vc + (size_t)g * a.ctx * HD;

    // 0. loads: this token's q, k, v rows, then the first keys' K rows and the first V tile
    constexpr int TOK = (3 * HD + kA1Threads - 1) / kA1Threads;
    float tok[TOK];
#pragma unroll
    for (int i = 0; i < TOK; i++) {
        const int f = min(tid + kA1Threads * i, 3 * HD - 1), r = f / HD, d = f % HD;
        tok[i] = r == 0 ? a.q[(size_t)h * HD + d] : (r == 1 ? a.k[(size_t)g * HD + d] : a.v[(size_t)g * HD + d]);
    }
    uint4 kr[KV4];
    {
        const int j = min(tid, max(pos - 1, 0));  // keys < pos come from the cache
#pragma unroll
        for (int i = 0; i < KV4; i++) kr[i] = *reinterpret_cast<const uint4*>(K + (size_t)j * HD + 8 * i);
    }
    uint4 vr[VT_LOADS];
#pragma unroll
    for (int i = 0; i < VT_LOADS; i++) {
        const int f = tid + kA1Threads * i, j = min(f / KV4, max(pos - 1, 0));
        vr[i] = *reinterpret_cast<const uint4*>(V + (size_t)j * HD + 8 * (f % KV4));
    }
    a1_fence();

    // 1. RoPE (NeoX, src/model.c:754-765) of q and k, then their RMSNorm (src/model.c:840-841)
#pragma unroll
    for (int i = 0; i < TOK; i++) {
        const int f = tid + kA1Threads * i;
        if (f < 3 * HD) row[f / HD][f % HD] = tok[i];
    }
    __syncthreads();
    const float* cs = a.rope_cos + (size_t)pos * half;
    const float* sn = a.rope_sin + (size_t)pos * half;
    static_assert(2 * HD <= kA1Threads, "one thread per q / k element");
    float rot = 0.f;
    if (tid < 2 * HD) {
        const int r = tid / HD, d = tid % HD;
        rot = row[r][d];
        if (d < half) rot = row[r][d] * cs[d] - row[r][d + half] * sn[d];
        else if (d < 2 * half) rot = row[r][d - half] * sn[d - half] + row[r][d] * cs[d - half];
    }
    __syncthreads();
    if (tid < 2 * HD) row[tid / HD][tid % HD] = rot;
    __syncthreads();
    if (wave < 2) {
        const float sum = hy_wave_seq_sq_sum(row[wave], HD, lane);
        if (lane == 0) stat[wave] = 1.0f / sqrtf(sum / (float)HD + a.eps);
    }
    __syncthreads();
    if (tid < 2 * HD) {
        const int r = tid / HD, d = tid % HD;
        const float y = row[r][d] * stat[r] * (r == 0 ? a.q_norm[d] : a.k_norm[d]);
        if (r == 0) row[0][d] = y;
        else kb[d] = hy_to_bf16(y);
    }
    for (int d = tid; d < HD; d += kA1Threads) vb[d] = hy_to_bf16(row[2][d]);
    __syncthreads();
    // the bf16 k, v of this position (src/model.c:842-847), stored once per KV head
    if (h % group == 0 && tid < HD) {
        const size_t off = ((size_t)g * a.ctx + pos) * HD + tid;
        a.kc[off] = kb[tid];
        a.vc[off] = vb[tid];
    }

    // 2. scores s_j = dot_bf16(q, K_j) * (1/sqrtf(hd)); key `pos` is this token's kb
    const float scale = 1.0f / sqrtf((float)HD);
    const float* qn = row[0];
    float lmax = -__builtin_inff();
    for (int p0 = 0; p0 < n; p0 += kA1Keys) {
        const int j = p0 + tid;
        if (p0 > 0) {
            const int jl = min(j, max(pos - 1, 0));
#pragma unroll
            for (int i = 0; i < KV4; i++) kr[i] = *reinterpret_cast<const uint4*>(K + (size_t)jl * HD + 8 * i);
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
            const float s = ((a0 + a1) + (a2 + a3)) * scale;
            sc[j] = s;
            lmax = fmaxf(lmax, s);
        }
    }
    // 3. softmax over positions: max (order-free), exp, sum in order, normalise
    lmax = hy_wave_max(lmax);
    if (lane == 0) red[wave] = lmax;
    __syncthreads();
    const float mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int j = tid; j < n; j += kA1Threads) sc[j] = hy_expf(sc[j] - mx);
    __syncthreads();
    if (wave == 0) {
        const float sum = hy_wave_seq_sum(sc, n, lane);
        if (lane == 0) stat[0] = 1.0f / sum;
    }
    __syncthreads();
    const float inv = stat[0];
    for (int j = tid; j < n; j += kA1Threads) sc[j] = sc[j] * inv;

    // 4. o[d] = sum_j p_j * V_j[d] in position order, from LDS tiles of V
    float o = 0.f;
    for (int t0 = 0; t0 < n; t0 += kA1Tile) {
        __syncthreads();  // previous tile consumed; probabilities visible
#pragma unroll
        for (int i = 0; i < VT_LOADS; i++) {
            const int f = tid + kA1Threads * i, jj = f / KV4, j = t0 + jj;
            const uint4 val = j == pos ? *reinterpret_cast<const uint4*>(vb + 8 * (f % KV4)) : vr[i];
            *reinterpret_cast<uint4*>(vt + (size_t)jj * HD + 8 * (f % KV4)) = val;
        }
        __syncthreads();
        if (t0 + kA1Tile < n) {  // next tile in flight while this one is summed
#pragma unroll
            for (int i = 0; i < VT_LOADS; i++) {
                const int f = tid + kA1Threads * i, j = min(t0 + kA1Tile + f / KV4, max(pos - 1, 0));
                vr[i] = *reinterpret_cast<const uint4*>(V + (size_t)j * HD + 8 * (f % KV4));
            }
        }
        if (tid < HD) {
            const int cnt = min(kA1Tile, n - t0);
            const float* pj = sc + t0;
            int jj = 0;
            for (; jj + 8 <= cnt; jj += 8) {
                float pv[8], vv[8];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    pv[k] = pj[jj + k];
                    vv[k] = hy_bf16(vt[(size_t)(jj + k) * HD + tid]);
                }
#pragma unroll
                for (int k = 0; k < 8; k++) o += pv[k] * vv[k];
            }
            for (; jj < cnt; jj++) o += pj[jj] * hy_bf16(vt[(size_t)jj * HD + tid]);
        }
    }
    if (tid < HD) a.ao[(size_t)h * HD + tid] = o;
}

size_t attn1_lds(int ctx) { return (size_t)ctx * sizeof(float); }

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
