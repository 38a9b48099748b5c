// Kernel launch descriptors and launchers (host-visible, C++ linkage, library-internal).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "hy_common.h"

namespace hy {

enum Kind : int { KIND_PANEL = 0, KIND_Q4K = 1, KIND_Q6K = 2, KIND_F16 = 3, KIND_F32 = 4, KIND_Q8_0 = 5, KIND_ANY = 7 };
enum Epi : int { EPI_STORE = 0, EPI_ADD = 1 };
enum Pro : int { PRO_NONE = 0, PRO_NORM = 1, PRO_QUANT = 2 };

// One weight matrix resident in HBM, in the layout its matvec kernel streams.
//   PANEL: w = codes [n][nb][64 B], ps = fp32 [n][nb]
//   Q4K:   w = reference blocks [n][nb][144 B]
//   Q6K:   planes, all indexed by block id n*nb+b: w = ql [..][128], w2 = qh [..][64],
//          sc = int8 scales [..][16], dh = f16 d [..] (same 210 bytes per block, aligned)
//   F16/F32: w = row tiles (hy_tile_offset): rows in groups of kRowTile, each group stored as
//          its rows' 16-byte pieces, piece by piece, so that the LM head (one thread per row,
//          all rows of a group stepping through their pieces together) reads contiguous memory
//   Q8_0:  the 34-byte blocks (f16 d, int8 qs[32]) split into two row-tiled arrays:
//          w = int8 weights [n][k], w2 = f16 scales [n][k / 32]
struct MvWeight {
    int kind, n, k, nb;
    int pshift, poff;
    const uint8_t* w;
    const uint8_t* w2;
    const int8_t* sc;
    const uint16_t* dh;
    const float* ps;
};

// Row-tiled layout of F16/F32 weights: byte b of row r sits at
//   ((r / kRowTile * (rowbytes / 16) + b / 16) * kRowTile + r % kRowTile) * 16 + b % 16,
// the last group padded with zero rows to kRowTile rows (rowbytes a multiple of 64).
constexpr int kRowTile = 256;
__host__ __device__ inline size_t hy_tile_offset(size_t r, size_t b, size_t rowbytes) {
    return ((r / kRowTile * (rowbytes / 16) + b / 16) * kRowTile + r % kRowTile) * 16 + b % 16;
}
__host__ __device__ inline size_t hy_tile_bytes(size_t n, size_t rowbytes) {
    return (n + kRowTile - 1) / kRowTile * kRowTile * rowbytes;
}

struct MvJob {
    MvWeight W;
    float* out;       // out[t * ldo + r]
    int ldo;
    int epi;          // EPI_STORE / EPI_ADD (out = out + acc, the reference's residual add)
    int rows_per_wg;  // tile height
    int wg_begin;     // first workgroup of this job in the grid
};

constexpr int kMaxJobs = 3;

struct MvLaunch {
    MvJob job[kMaxJobs];
    int njobs;
    int pair;              // 1: job[0]=gate, job[1]=up share tiles; job[0].out <- silu(g)*u
    int nt;
    const HyQ8K* act;      // PRO_NONE: activations [nt][nb]
    const float* x;        // PRO_NORM: h [K]; PRO_QUANT: vector [K] (nt == 1 for both)
    const float* norm_w;   // PRO_NORM weights [K]
    float eps;
    int K;                 // input dim of all jobs
    int segs;              // 16-byte segments per thread (1, 2 or 4)
    int threads;           // workgroup size: 256 (PRO_NONE / PRO_NORM) or 1024 (PRO_NORM / PRO_QUANT)
};

// Which (template) variant a matvec launch uses; decided on the host.
int mv_segments_per_block(int kind);

hipError_t launch_quantize_q8k(const float* x, int ldx, HyQ8K* act, int K, int nt, hipStream_t s);
hipError_t launch_rmsnorm_q8k(const float* h, const float* w, float eps, int H, int nt, float* xn_out,
                              HyQ8K* act_out, hipStream_t s);
hipError_t launch_matvec(const MvLaunch& L, int pro, int grid, hipStream_t s);
size_t matvec_lds_bytes(const MvLaunch& L, int pro);

// Single-token matvec of the fused decode step (k_mv1, hy_decode_mv.hip). Each half-wavefront
// owns one weight row per iteration; a lane owns the same 16-byte segment positions in every
// row it visits, so its slice of the Q8_K activation stays in registers.
struct Mv1Job {
    MvWeight W;
    float* out;      // out[r]
    int epi;         // EPI_STORE / EPI_ADD
    int wg_begin;    // first workgroup of this job in the grid
};

struct Mv1Launch {
    Mv1Job job[kMaxJobs];
    int njobs;
    int pair;              // job[0] = gate, job[1] = up of equal shape: job[0].out[r] = silu(g_r) * u_r
    int rows_per_wg;       // rows (pair: row pairs) per workgroup
    const HyQ8K* act;      // PRO_NONE: Q8_K activation blocks [K / 256]
    const float* x;        // PRO_NORM: h [K]; PRO_QUANT: fp32 input [K]
    const float* norm_w;   // PRO_NORM weights [K]
    float eps;
    int K;
    unsigned long long* slots;  // optional: the greedy argmax over rows < n_arg, one key per workgroup
    int n_arg;
    int grid;              // set by launch_mv1: its workgroups (argmax slots written)
};

// Builds and launches k_mv1 for jobs of one kind class with K = 2048 or 6144; returns
// hipErrorNotSupported when the shapes fall outside what k_mv1 handles (the caller then uses
// launch_matvec).
hipError_t launch_mv1(Mv1Launch& L, int pro, hipStream_t s);

// Multi-token GEMM of panel weights on int8 MFMA (k_gemm_panel, hy_prefill.hip): out[t * ldo + r]
// for nt tokens of Q8_K activations [nt][K / 256], bit-identical to nt single-token matvecs.
struct GemmJob {
    MvWeight W;
    float* out;
    int ldo;
    int epi;         // EPI_STORE / EPI_ADD
    int tile_begin;  // first row tile of this job in the grid (set by the launcher)
    const HyQ8K* act;  // this job's activations [nt][nb] (null: the launch's act and nt)
    int nt;
};

// Chunks in flight in the pipelined prefill (hymt2_hip_gen_prefill): the chunk kernels and the
// GEMM take tables of up to this many chunks (the GEMM three weights each) in one launch.
constexpr int kPipeMax = 8;
constexpr int kGemmPipeJobs = 3 * kPipeMax;

template <int NJ>
struct GemmLaunchT {
    GemmJob job[NJ];
    int njobs;
    int pair;              // jobs (2p, 2p + 1) = gate, up of equal shape: job[2p].out = silu(g) * u
    int nt;
    const HyQ8K* act;      // [nt][nb]
    int nb;                // set by the launcher
};
using GemmLaunch = GemmLaunchT<kMaxJobs>;
using GemmPipeLaunch = GemmLaunchT<kGemmPipeJobs>;
// hipErrorNotSupported for weights that are not panels of one K (the caller then uses
// launch_matvec).
hipError_t launch_gemm_panel(GemmLaunch& L, hipStream_t s);
hipError_t launch_gemm_panel(GemmPipeLaunch& L, hipStream_t s);

struct AttnArgs {
    float* q;              // [nt][qdim]
    const float* k;        // [nt][kvdim]
    const float* v;        // [nt][kvdim]
    uint16_t* kc;          // layer base of K cache [kv_heads][ctx][hdim]
    uint16_t* vc;          // layer base of V cache
    float* ao;             // [nt][qdim]
    const float* q_norm;   // [hdim]
    const float* k_norm;   // [hdim]
    const float* rope_cos; // [ctx][rope_half]
    const float* rope_sin;
    const int* pos_dev;    // optional: pos0 read from device memory (graph replay)
    int pos0, nt, heads, kv_heads, hdim, rope_half, ctx;
    float eps;
    HyQ8K* act_out;        // optional [nt][qdim / 256]: Q8_K blocks of ao, where attention_quantizes()
};
hipError_t launch_rope_norm_store(const AttnArgs& a, hipStream_t s);
// True when launch_attention also writes a.act_out (the chunk kernel's head group covers whole
// Q8_K blocks); otherwise the caller quantizes ao itself.
bool attention_quantizes(const AttnArgs& a);

hipError_t launch_attention(const AttnArgs& a, hipStream_t s);

// Several chunks in one launch (the pipelined prefill): job j owns the grid's token rows
// row0[j] .. row0[j] + nt_j - 1 (row0[0] = 0, increasing); each workgroup finds its job by row.
struct PipeAttn {
    AttnArgs a[kPipeMax];
    int row0[kPipeMax];
    int njobs;
};
struct PipeNorm {
    const float* h[kPipeMax];  // [nt_j][2048]
    const float* w[kPipeMax];  // norm weights [2048]
    HyQ8K* act[kPipeMax];      // [nt_j][8]
    int row0[kPipeMax];
    int njobs;
    float eps;
};
struct PipeQuant {
    const float* x[kPipeMax];  // [nt_j][ldx]
    HyQ8K* act[kPipeMax];      // [nt_j][K / 256]
    int row0[kPipeMax];
    int njobs, ldx, K;
};
// The job of grid row `row` in such a launch (uniform: scalar compares against the table).
__device__ __forceinline__ int pipe_job(const int* row0, int njobs, int row) {
    int j = 0;
#pragma unroll
    for (int q = 1; q < kPipeMax; q++)
        if (q < njobs && row >= row0[q]) j = q;
    return j;
}
// rows: the total token rows of the jobs. The attention form is the chunk kernel's only
// (attention_quantizes() for every job, ctx within its LDS rows): hipErrorNotSupported otherwise.
hipError_t launch_rope_norm_store(const PipeAttn& J, int rows, hipStream_t s);
hipError_t launch_attention(const PipeAttn& J, int rows, hipStream_t s);
hipError_t launch_rmsnorm_q8k(const PipeNorm& J, int rows, hipStream_t s);  // hidden 2048 only
hipError_t launch_quantize_q8k(const PipeQuant& J, int rows, hipStream_t s);

// Single-token attention, one workgroup per query head (k_attn1, hy_attn_decode.hip): RoPE
// and RMSNorm of q and k, the bf16 KV store at the position, softmax attention over positions
// 0..pos, fp32 output row per head into ao (quantized by the o-projection).
constexpr int kA1MaxCtx = 4096;
struct Attn1Args {
    const float* q;        // [qdim] fp32, before RoPE
    const float* k;        // [kvdim]
    const float* v;        // [kvdim]
    uint16_t* kc;          // layer base of K cache [kv_heads][ctx][hdim]
    uint16_t* vc;
    const float* q_norm;
    const float* k_norm;
    const float* rope_cos;
    const float* rope_sin;
    const int* pos_dev;    // optional: position read from device memory (graph replay)
    const float* rope_cur; // with pos_dev: that position's RoPE row (cos[half], sin[half])
    int pos0;
    float* ao;             // [qdim] attention output
    int heads, kv_heads, hdim, rope_half, ctx;
    float eps;
    // split form only (launch_attn_split): scores and per-segment maxima of each query head
    float* sc;             // [heads][sc_stride] fp32 scores (written by k_attn_scores, only read after)
    float* segmax;         // [heads][seg_stride] maximum score of each kSplitMaxSeg positions
    int sc_stride, seg_stride;
};
hipError_t launch_attn1(const Attn1Args& a, hipStream_t s);

// Split single-token attention for long rows (hy_attn_decode.hip): k_attn_scores spreads the
// scores of each KV head's query heads over workgroups of kSplitSeg positions (with RoPE, the
// q/k norms and the KV store), then k_attn_out (one workgroup per query head and 64 output
// dimensions) forms the softmax and the output. Any context length; bit-identical to k_attn1.
constexpr int kSplitSeg = 64;     // positions per score workgroup segment (a key per pair of lanes)
constexpr int kSplitMaxSeg = 32;  // positions per segment maximum (one wavefront's keys)
constexpr int kSplitWin = 4096;   // positions of p_j held in LDS at a time
constexpr int kSplitMaxGroup = 16;
inline int split_sc_stride(int ctx) { return (ctx + kSplitSeg - 1) / kSplitSeg * kSplitSeg; }
inline int split_seg_stride(int ctx) { return (ctx + kSplitSeg - 1) / kSplitSeg * (kSplitSeg / kSplitMaxSeg); }
hipError_t launch_attn_split(const Attn1Args& a, hipStream_t s);

struct HeadArgs {
    MvWeight W;            // F16, F32 or Q8_0 row tiles
    const float* h;        // last token's hidden state [K]
    const float* norm_w;   // output norm
    float eps;
    float* logits;         // [n]
    unsigned long long* argmax_key;  // optional fused argmax over rows < n_arg, by atomicMax into one key
    int n_arg;
    unsigned long long* slots;       // or: one key per workgroup (slot = workgroup, head_grid of them)
};
hipError_t launch_head(const HeadArgs& a, hipStream_t s);
constexpr int kHeadThreads = 256;  // LM head rows per workgroup (one per thread; 128 measured slower)
inline int head_grid(int n) { return (n + kHeadThreads - 1) / kHeadThreads; }
// Argmax slots of the device loop: one per workgroup of the LM head kernel that writes them.
constexpr int kArgSlots = 8192;

struct FinishArgs {
    const unsigned long long* slots;  // the head's per-workgroup argmax keys
    int nslots;
    int* ids;              // token ids [n_total]
    int* step;             // device step counter (position of the token just processed)
    int n_prompt;
    MvWeight E;            // token embedding [vocab][H]: F16 / F32 / Q8_0 / Q4_K / Q6_K
    float* h;              // next step's input [H]
    int H;
    int n_total;
    const float* rope_cos; // RoPE tables [ctx][half]; the next position's row is copied to
    const float* rope_sin; // rope_cur (cos then sin) for the next step's attention
    float* rope_cur;
    int rope_half, ctx;
    // stop ids of the loop (tok_is_stop, src/tokenizer.c:179): stop[0..kStopIds) (-1 pads), then
    // stop[kStopIds] = the first position whose generated id is one of them (INT_MAX: none yet);
    // stop_host (host-mapped) receives the same position when it is set
    int* stop;
    int* stop_host;
};
constexpr int kStopIds = 8;
hipError_t launch_finish(const FinishArgs& a, hipStream_t s);
// True for the embedding kinds embed_row dequantizes (src/kernels.c:1304-1329).
inline bool embed_kind(int kind) {
    return kind == KIND_F16 || kind == KIND_F32 || kind == KIND_Q8_0 || kind == KIND_Q4K || kind == KIND_Q6K;
}
hipError_t launch_embed(const int* ids, const int* step, const MvWeight& E, float* h, int H, hipStream_t s);
hipError_t launch_embed_rows(const int* ids, int first, int nt, const MvWeight& E, float* h, int H, hipStream_t s);
hipError_t launch_set_int(int* p, int v, hipStream_t s);

// The greedy argmax of v[0 .. n) as one key per 256-element workgroup into slots (argmax_grid(n) slots).
inline int argmax_grid(int n) { return (n + 255) / 256; }
hipError_t launch_argmax(const float* v, int n, unsigned long long* slots, hipStream_t s);
hipError_t launch_silu_mul(float* g, const float* u, int n, hipStream_t s);
hipError_t launch_selftest(const void* src, float* dst, int n, int what, hipStream_t s);
hipError_t launch_selftest_sqsum(const float* x, int n, int m, float* out, int method, hipStream_t s);
hipError_t launch_selftest_mfma(const float* a, const float* b, float* out, int nw, hipStream_t s);

}  // namespace hy
