// Host side of the HIP backend: the hy_device_ops vtable the reference host calls
// (src/device.h:70-80), built MI355X-first: weights resident in HBM in kernel-friendly layouts,
// one HIP stream per context, single-token forwards replayed from a captured hipGraph, one
// host synchronisation per fused_forward, and a device-resident greedy loop.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unistd.h>
#include <vector>

#include "../../include/hymt2_hip.h"
#include "hy_kernels.h"

using namespace hy;

// ----------------------------------------------------------------------------------- ABI

static_assert(sizeof(hymt2_weight) == 64, "weight_t size");
static_assert(offsetof(hymt2_weight, row_bytes) == 24 && offsetof(hymt2_weight, pk) == 32 &&
                  offsetof(hymt2_weight, ps) == 40 && offsetof(hymt2_weight, pshift) == 48 &&
                  offsetof(hymt2_weight, gpu) == 56,
              "weight_t layout");
static_assert(sizeof(hymt2_q8k_block) == 576 && sizeof(HyQ8K) == 576, "q8k_block size");
static_assert(sizeof(hymt2_fused_layer) == 88, "hy_fused_layer size");
static_assert(sizeof(hymt2_fused_args) == 112 && offsetof(hymt2_fused_args, eps) == 48 &&
                  offsetof(hymt2_fused_args, layers) == 56 && offsetof(hymt2_fused_args, logits) == 104,
              "hy_fused_args layout");
static_assert(sizeof(hymt2_device_ops) == 64, "hy_device_ops size");

// The reference host's wrapper (src/device.c:25-35). Weak: absent when this library is loaded
// on its own, in which case hy_cuda_create reports that the host is missing.
extern "C" hy_device* hy_device_wrap(int kind, const char* name, void* impl, const hymt2_device_ops* ops,
                                     bool software) __attribute__((weak));
static constexpr int kDevKindCuda = 2;  // HY_DEV_CUDA, src/device.h:15-21

// ggml type codes, src/internal.h:46
enum { GT_F32 = 0, GT_F16 = 1, GT_Q8_0 = 8, GT_Q4_K = 12, GT_Q6_K = 14, GT_Q2_0C = 40, GT_STQ1_0 = 43 };

struct Ctx;

struct DW {  // hy_dweight
    Ctx* c = nullptr;
    int gtype = 0;
    MvWeight mw{};
    void* mem = nullptr;
    size_t bytes = 0;
    // weight_out: pinned, device-mapped output rows [HY_MAX_BATCH][n] (allocated on first use);
    // matmul writes them from the kernels directly when the host passes them as the output
    float* op_host = nullptr;
    float* op_dev = nullptr;
};

// Input staging layout (device in_dev and pinned in_host): the position, its RoPE row, then the
// hidden rows of the chunk at kInH.
constexpr size_t kInH = 2048;

// Single-token forwards at positions from here on use the split attention (launch_attn_split).
constexpr int kSplitFromDefault = 448;
// Device-loop steps captured in one graph: each graph launch costs about 8.5 us of idle GPU
// between the previous graph's last kernel and the next graph's first.
constexpr int kStepsPerGraph = 8;

struct Fused {
    int n_layer = 0, hidden = 0, ffn = 0, heads = 0, kv_heads = 0, hdim = 0, qdim = 0, kvdim = 0, ctx = 0,
        rope_half = 0;
    float eps = 0.f;
    char* in_dev = nullptr;   // [pos int | pad to 64 B][RoPE row of pos: cos, sin | pad to kInH]
                              // [HY_MAX_CHUNK * hidden floats]
    char* in_host = nullptr;  // pinned staging of the same layout
    float* d_h = nullptr;
    int* d_pos = nullptr;
    float* d_rope = nullptr;  // RoPE row of d_pos (single-token graphs)
    size_t in_bytes = 0;
    float *q = nullptr, *k = nullptr, *v = nullptr, *ao = nullptr, *g = nullptr, *u = nullptr, *logits = nullptr;
    HyQ8K *act_h = nullptr, *act_q = nullptr, *act_f = nullptr;
    float *rope_c = nullptr, *rope_s = nullptr, *out_norm = nullptr, *norms = nullptr;
    uint16_t *kc = nullptr, *vc = nullptr;
    size_t logits_cap = 0;
    unsigned long long* slots = nullptr;  // argmax keys of the LM head, one per workgroup (kArgSlots)
    int head_slots = 0;                   // the slots the last enqueued head with argmax writes
    int* ids = nullptr;
    int ids_cap = 0;
    int gen_total = 0;   // positions of the current device loop (0: no loop begun)
    int gen_steps = 0;   // steps enqueued so far (positions processed, the reused prefix included)
    int gen_prompt = 0, gen_vocab = 0;
    int gen_keep = 0;    // prompt positions whose K/V the loop reused (its first step's position)
    MvWeight gen_embd{};  // embedding of the current device loop
    // stop ids of the device loop and the first stop position (FinishArgs::stop), and the
    // host-mapped copy of that position the host loop polls
    int* stop = nullptr;
    int* stop_host = nullptr;
    int* stop_host_dev = nullptr;
    // the ids whose K/V the cache holds after the last hymt2_hip_generate_ids call (positions
    // 0 .. cache_n - 1), and what they were computed with; any other writer of the cache
    // (fused_forward, the other device-loop entry points) sets cache_n to 0
    std::vector<int> cache_tok;
    int cache_n = 0;
    std::vector<const void*> cache_sig;
    // attention scratch of the split form (launch_attn_split): scores [heads][sc_stride] and
    // segment maxima [heads][seg_stride]
    float *sc = nullptr, *segmax = nullptr;
    // captured single-token graphs, [0] with the one-kernel attention (k_attn1), [1] with the
    // split form; a forward at position p replays [split_at(p)]
    hipGraphExec_t g_fwd[2] = {nullptr, nullptr}, g_step[2] = {nullptr, nullptr};
    hipGraphExec_t g_steps[2] = {nullptr, nullptr};  // kStepsPerGraph steps of the device loop in one graph
    std::vector<const void*> sig_fwd[2], sig_step;
    // chunk slots of the pipelined prefill (allocated on first use): kPipeMax slots of
    // HY_MAX_CHUNK token rows each, slot-major
    float *p_h = nullptr, *p_q = nullptr, *p_k = nullptr, *p_v = nullptr, *p_ao = nullptr, *p_g = nullptr;
    HyQ8K *p_act_h = nullptr, *p_act_q = nullptr, *p_act_f = nullptr;
    float* norm_ptr(int li, int which) const {  // 0 attn, 1 ffn, 2 q, 3 k
        const size_t per = 2 * (size_t)hidden + 2 * (size_t)hdim;
        float* base = norms + per * li;
        return which == 0 ? base : which == 1 ? base + hidden : which == 2 ? base + 2 * hidden : base + 2 * hidden + hdim;
    }
};

struct Ctx {
    int dev = 0;
    hipStream_t s = nullptr;
    bool broken = false;
    std::string err;
    void* act = nullptr;
    size_t act_cap = 0;
    float* out = nullptr;
    size_t out_cap = 0;
    Fused* f = nullptr;
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    hipEvent_t ring[2] = {nullptr, nullptr};  // the last two decode launches of hymt2_hip_generate_ids
    uint8_t* scratch = nullptr;  // this device's address of `scratch` (hymt2_hip_matmul_static), or null
    int split_from = kSplitFromDefault;  // single-token attention at positions >= this: split form
    int pipe_depth = kPipeMax;           // chunks in flight in gen_prefill (1: one chunk after another)
};

// Whether the single-token forward at position pos uses the split attention: long rows, and
// every shape the one-kernel form (k_attn1: head dim 64 or 128, ctx <= kA1MaxCtx) does not take.
static bool split_at(const Ctx* c, const Fused* f, int pos) {
    return pos >= c->split_from || (f->hdim != 64 && f->hdim != 128) || f->ctx > kA1MaxCtx;
}

// Device staging of hymt2_hip_matmul_static, the per-op entry point that allocates nothing: the
// Q8_K activation blocks, then the outputs that go back by copy. Every GPU the library runs on
// holds one copy of it until the process ends; all calls on one GPU share that copy (calls that
// overlap on one GPU race on it). In host code the name is a host-side stand-in: kernels and
// copies use the device address hipGetSymbolAddress returns, kept per device in
// g_scratch_addr and per context in Ctx::scratch.
constexpr size_t kScratchBytes = 16u << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
static uint8_t* g_scratch_addr[kMaxDevices];
static std::mutex g_scratch_mu;

// This device's address of `scratch`, looked up once per device with that device current.
static uint8_t* scratch_address(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        g_scratch_addr[dev] = static_cast<uint8_t*>(p);
    }
    return g_scratch_addr[dev];
}

static void set_err(Ctx* c, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    c->err = buf;
    if (getenv("HYMT2_VERBOSE")) fprintf(stderr, "[hymt2-hip] %s\n", buf);
}

#define HIPCHK(c, x)                                                                  \
    do {                                                                              \
        hipError_t e_ = (x);                                                          \
        if (e_ != hipSuccess) {                                                       \
            set_err((c), "%s failed: %s (%s:%d)", #x, hipGetErrorString(e_), __FILE__, __LINE__); \
            (c)->broken = true;                                                       \
            return false;                                                             \
        }                                                                             \
    } while (0)

template <typename T>
static bool dalloc(Ctx* c, T** p, size_t bytes) {
    void* q = nullptr;
    hipError_t e = hipMalloc(&q, bytes ? bytes : 64);
    if (e != hipSuccess) {
        set_err(c, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
        return false;
    }
    *p = static_cast<T*>(q);
    return true;
}

// ----------------------------------------------------------------------------------- upload

// Kinds the per-op matmul runs: the reference multiplies them with the host's Q8_K activations.
static bool quant_kind(int kind) { return kind == KIND_PANEL || kind == KIND_Q4K || kind == KIND_Q6K; }

// True when the host will not take the fused path: HYMT2_FUSED=0/off/no forbids it
// (src/model.c:330-333). The per-op matmul receives only Q8_K activations, so without the fused
// path a weight that takes fp32 activations (F16, F32, Q8_0: the LM head) is declined at upload
// and the host computes it on the CPU, as it does with the reference CUDA backend
// (src/cuda.c:209-212). Accepting it would make the host's first matmul on it fail and turn the
// device off for the whole run (src/model.c:674-681).
static bool fused_forbidden() {
    const char* fe = getenv("HYMT2_FUSED");
    return fe && (!strcmp(fe, "0") || !strcmp(fe, "off") || !strcmp(fe, "no"));
}

// Q6_K blocks (210 B, src/internal.h:23: ql[128] qh[64] scales[16] d) -> four aligned planes of
// the same bytes, so every lane issues 16-byte loads.
static void q6k_to_planes(const uint8_t* src, size_t nblk, uint8_t* ql, uint8_t* qh, int8_t* sc, uint16_t* d) {
    for (size_t i = 0; i < nblk; i++) {
        const uint8_t* b = src + i * 210;
        memcpy(ql + i * 128, b, 128);
        memcpy(qh + i * 64, b + 128, 64);
        memcpy(sc + i * 16, b + 192, 16);
        memcpy(d + i, b + 208, 2);
    }
}

static hy_dweight* hip_upload(void* impl, const hymt2_weight* w) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || !w || w->k <= 0 || w->n <= 0) return nullptr;
    DW* d = new DW();
    d->c = c;
    d->gtype = w->type;
    MvWeight& m = d->mw;
    m.n = w->n;
    m.k = w->k;
    const size_t n = (size_t)w->n;
    std::vector<uint8_t> host;
    // row lengths whole blocks of the type: STQ1_0 256 weights a block, Q2_0C 512
    // (src/model.c:138, src/kernels.c:121); the panel then has k / 256 pieces a row
    if ((w->type == GT_STQ1_0 || w->type == GT_Q2_0C) && w->pk && w->ps && w->k % (w->type == GT_Q2_0C ? 512 : 256) == 0) {
        m.kind = KIND_PANEL;
        m.nb = w->k / 256;
        m.pshift = w->pshift;
        m.poff = w->poff;
        const size_t cb = n * m.nb * 64, sb = n * m.nb * 4;
        d->bytes = cb + sb;
        host.resize(d->bytes);
        memcpy(host.data(), w->pk, cb);
        memcpy(host.data() + cb, w->ps, sb);
    } else if (w->type == GT_Q4_K && w->k % 256 == 0) {
        m.kind = KIND_Q4K;
        m.nb = w->k / 256;
        d->bytes = n * m.nb * 144;
        host.assign(w->data, w->data + d->bytes);
    } else if (w->type == GT_Q6_K && w->k % 256 == 0) {
        m.kind = KIND_Q6K;
        m.nb = w->k / 256;
        const size_t nblk = n * m.nb;
        d->bytes = nblk * 210;
        host.resize(d->bytes);
        q6k_to_planes(w->data, nblk, host.data(), host.data() + nblk * 128,
                      reinterpret_cast<int8_t*>(host.data() + nblk * 192),
                      reinterpret_cast<uint16_t*>(host.data() + nblk * 208));
    } else if ((w->type == GT_F16 || w->type == GT_F32 || w->type == GT_Q8_0) && fused_forbidden()) {
        set_err(c, "upload: type %d takes fp32 activations and HYMT2_FUSED forbids the fused path", w->type);
        delete d;
        return nullptr;
    } else if ((w->type == GT_F16 && w->k % 32 == 0) || (w->type == GT_F32 && w->k % 16 == 0)) {
        // row tiles (hy_tile_offset): the LM head reads each group's rows piece by piece
        m.kind = w->type == GT_F16 ? KIND_F16 : KIND_F32;
        m.nb = w->k / 256;
        const size_t rowb = (size_t)w->k * (w->type == GT_F16 ? 2 : 4);
        d->bytes = hy_tile_bytes(n, rowb);
        host.assign(d->bytes, 0);
        for (size_t r = 0; r < n; r++)
            for (size_t b = 0; b < rowb; b += 16) memcpy(host.data() + hy_tile_offset(r, b, rowb), w->data + r * rowb + b, 16);
    } else if (w->type == GT_Q8_0 && w->k % 256 == 0) {
        // 34-byte blocks (f16 d, int8 qs[32], src/internal.h:22) -> row-tiled int8 weights and
        // row-tiled f16 scales, read by the LM head one thread per row
        m.kind = KIND_Q8_0;
        m.nb = w->k / 256;
        const size_t qrow = (size_t)w->k, drow = (size_t)w->k / 16, qb = hy_tile_bytes(n, qrow);
        d->bytes = qb + hy_tile_bytes(n, drow);
        host.assign(d->bytes, 0);
        for (size_t r = 0; r < n; r++) {
            const uint8_t* row = w->data + r * (size_t)(w->k / 32) * 34;
            for (int b = 0; b < w->k / 32; b++) {
                memcpy(host.data() + qb + hy_tile_offset(r, 2 * (size_t)b, drow), row + 34 * b, 2);
                for (int piece = 0; piece < 2; piece++)
                    memcpy(host.data() + hy_tile_offset(r, 32 * (size_t)b + 16 * piece, qrow), row + 34 * b + 2 + 16 * piece, 16);
            }
        }
    } else {
        set_err(c, "upload: unsupported weight type %d (k=%d, panel=%d)", w->type, w->k, w->pk != nullptr);
        delete d;
        return nullptr;
    }
    if (!dalloc(c, &d->mem, d->bytes) ||
        hipMemcpy(d->mem, host.data(), d->bytes, hipMemcpyHostToDevice) != hipSuccess) {
        if (d->mem) (void)hipFree(d->mem);
        set_err(c, "upload: device copy of %zu bytes failed", d->bytes);
        delete d;
        return nullptr;
    }
    uint8_t* base = static_cast<uint8_t*>(d->mem);
    m.w = base;
    if (m.kind == KIND_PANEL) {
        m.ps = reinterpret_cast<const float*>(base + n * m.nb * 64);
    } else if (m.kind == KIND_Q6K) {
        const size_t nblk = n * m.nb;
        m.w2 = base + nblk * 128;
        m.sc = reinterpret_cast<const int8_t*>(base + nblk * 192);
        m.dh = reinterpret_cast<const uint16_t*>(base + nblk * 208);
    } else if (m.kind == KIND_Q8_0) {
        m.w2 = base + hy_tile_bytes(n, (size_t)w->k);
    }
    return reinterpret_cast<hy_dweight*>(d);
}

static void free_graphs(Fused* f);

// Frees a device weight. The context's captured graphs may name it (their signatures hold
// weight handles, and a later upload can reuse the address), so they are dropped too.
static void hip_release(hy_dweight* w) {
    DW* d = reinterpret_cast<DW*>(w);
    if (!d) return;
    if (d->c && d->c->f) {
        if (d->c->s) (void)hipStreamSynchronize(d->c->s);
        free_graphs(d->c->f);
    }
    if (d->mem) (void)hipFree(d->mem);
    if (d->op_host) (void)hipHostFree(d->op_host);
    delete d;
}

static bool hip_is_sw(const void*) { return false; }

// weight_out (src/device.h:76; the reference's cu_weight_out, src/cuda.c:107): a host-visible
// output buffer of HY_MAX_BATCH rows for this weight. The host hands it back to matmul as the
// output (gpu_out, src/model.c:662-667), and matmul's kernels then write it over PCIe directly:
// no device output buffer and no copy. NULL (the host then uses its own buffer) for weights the
// per-op path does not run, or when the pinned allocation fails.
static float* hip_weight_out(hy_dweight* w) {
    DW* d = reinterpret_cast<DW*>(w);
    if (!d || !quant_kind(d->mw.kind)) return nullptr;
    if (!d->op_host) {
        void* p = nullptr;
        const size_t bytes = (size_t)d->mw.n * HY_MAX_BATCH * sizeof(float);
        if (hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) return nullptr;
        void* pd = nullptr;
        if (hipHostGetDevicePointer(&pd, p, 0) != hipSuccess) {
            (void)hipHostFree(p);
            return nullptr;
        }
        d->op_host = static_cast<float*>(p);
        d->op_dev = static_cast<float*>(pd);
    }
    return d->op_host;
}

// ----------------------------------------------------------------------------------- matvec

struct JobSpec {
    const DW* w;
    float* out;
    int ldo;
    int epi;
};

// Tile the jobs over workgroups of `threads` lanes: the smallest segments-per-thread whose grid
// stays within a few resident workgroups per CU.
static bool build_launch(const JobSpec* js, int njobs, bool pair, int nt, int threads, MvLaunch& L, int& grid) {
    memset(&L, 0, sizeof L);
    L.njobs = njobs;
    L.pair = pair ? 1 : 0;
    L.nt = nt;
    L.threads = threads;
    const int K = js[0].w->mw.k;
    const int max_wgs = threads == 1024 ? 128 : 1024;
    for (int segs : {1, 2, 4}) {
        int wgs = 0;
        bool ok = true;
        for (int j = 0; j < njobs && ok; j++) {
            const MvWeight& m = js[j].w->mw;
            const int spr = m.nb * mv_segments_per_block(m.kind) * (pair ? 2 : 1);
            const int rpw = (threads * segs) / spr;
            if (rpw < 1) ok = false;
            L.job[j].rows_per_wg = rpw;
            L.job[j].wg_begin = wgs;
            if (!pair || j == 0) wgs += (m.n + rpw - 1) / rpw;
        }
        if (!ok) continue;
        L.segs = segs;
        grid = wgs;
        if (wgs <= max_wgs) break;
    }
    if (!L.segs) return false;
    for (int j = 0; j < njobs; j++) {
        L.job[j].W = js[j].w->mw;
        L.job[j].out = js[j].out;
        L.job[j].ldo = js[j].ldo;
        L.job[j].epi = js[j].epi;
        if (js[j].w->mw.k != K || !quant_kind(js[j].w->mw.kind)) return false;
    }
    if (pair) {
        if (njobs != 2 || js[0].w->mw.kind != js[1].w->mw.kind || js[0].w->mw.n != js[1].w->mw.n) return false;
        L.job[1].rows_per_wg = L.job[0].rows_per_wg;
        L.job[1].wg_begin = 0;
    }
    L.K = K;
    return true;
}

struct MvOpts {
    int pro = PRO_NONE;
    int threads = 256;
    const HyQ8K* act = nullptr;
    const float* x = nullptr;
    const float* norm_w = nullptr;
    float eps = 0.f;
};

static bool run_matvec(Ctx* c, const JobSpec* js, int njobs, bool pair, int nt, const MvOpts& o) {
    MvLaunch L;
    int grid = 0;
    if (!build_launch(js, njobs, pair, nt, o.threads, L, grid)) {
        set_err(c, "matvec: unsupported job combination");
        return false;
    }
    L.act = o.act;
    L.x = o.x;
    L.norm_w = o.norm_w;
    L.eps = o.eps;
    HIPCHK(c, launch_matvec(L, o.pro, grid, c->s));
    return true;
}

// One token (nt == 1): the decode matvec k_mv1 where its shapes apply (K = 2048 / 6144, one
// kind class), else the general kernel.
static bool run_mv1(Ctx* c, const JobSpec* js, int njobs, bool pair, const MvOpts& o) {
    Mv1Launch L;
    memset(&L, 0, sizeof L);
    L.njobs = njobs;
    L.pair = pair ? 1 : 0;
    for (int j = 0; j < njobs; j++) {
        L.job[j].W = js[j].w->mw;
        L.job[j].out = js[j].out;
        L.job[j].epi = js[j].epi;
    }
    L.act = o.act;
    L.x = o.x;
    L.norm_w = o.norm_w;
    L.eps = o.eps;
    const hipError_t e = launch_mv1(L, o.pro, c->s);
    if (e == hipErrorNotSupported) return run_matvec(c, js, njobs, pair, 1, o);
    HIPCHK(c, e);
    return true;
}

// Several tokens: panel weights go to the int8-MFMA GEMM from kGemmMinTokens + 1 tokens (the
// reference host's 16-token batches among them); otherwise (and for Q4_K / Q6_K) the general
// matvec kernel runs over groups of at most HY_MAX_BATCH tokens. Both give every token the
// single-token result. The threshold as measured (a fused_forward of the config-3 model, matvec
// against GEMM: 16 tokens 3.27 -> 1.95-2.01 ms, 8 tokens 2.34 -> 1.91-1.97, 4 tokens equal,
// 2 tokens 1.71-1.78 against 1.87-1.92 ms)
constexpr int kGemmMinTokens = 4;

static bool run_multi(Ctx* c, const JobSpec* js, int njobs, bool pair, int nt, const MvOpts& o) {
    if (nt > kGemmMinTokens && o.pro == PRO_NONE) {
        GemmLaunch G;
        memset(&G, 0, sizeof G);
        G.njobs = njobs;
        G.pair = pair ? 1 : 0;
        G.nt = nt;
        G.act = o.act;
        for (int j = 0; j < njobs; j++) {
            G.job[j].W = js[j].w->mw;
            G.job[j].out = js[j].out;
            G.job[j].ldo = js[j].ldo;
            G.job[j].epi = js[j].epi;
        }
        const hipError_t e = launch_gemm_panel(G, c->s);
        if (e != hipErrorNotSupported) {
            HIPCHK(c, e);
            return true;
        }
    }
    if (nt <= HY_MAX_BATCH || o.pro != PRO_NONE) return run_matvec(c, js, njobs, pair, nt, o);
    const int nb = js[0].w->mw.nb;
    for (int t0 = 0; t0 < nt; t0 += HY_MAX_BATCH) {
        JobSpec g[kMaxJobs];
        for (int j = 0; j < njobs; j++) {
            g[j] = js[j];
            g[j].out = js[j].out + (size_t)t0 * js[j].ldo;
        }
        MvOpts og = o;
        og.act = o.act + (size_t)t0 * nb;
        if (!run_matvec(c, g, njobs, pair, std::min(HY_MAX_BATCH, nt - t0), og)) return false;
    }
    return true;
}

static bool ensure_scratch(Ctx* c, size_t act_bytes, size_t out_bytes) {
    if (act_bytes > c->act_cap) {
        if (c->act) (void)hipFree(c->act);
        c->act = nullptr;
        c->act_cap = 0;
        if (!dalloc(c, &c->act, act_bytes)) return false;
        c->act_cap = act_bytes;
    }
    if (out_bytes > c->out_cap) {
        if (c->out) (void)hipFree(c->out);
        c->out = nullptr;
        c->out_cap = 0;
        if (!dalloc(c, &c->out, out_bytes)) return false;
        c->out_cap = out_bytes;
    }
    return true;
}

// One per-op group on the given device staging: the host's Q8_K activations are copied to act,
// each weight's output goes to its pinned weight_out rows when the host passed those (written by
// the kernels directly), else to `out` and back to the host's buffer; one synchronisation.
static bool matmul_group(Ctx* c, hy_dweight* const* ws, float* const* outs, int cnt, const hymt2_q8k_block* xq, int nt,
                         HyQ8K* act, float* out) {
    const DW* w0 = reinterpret_cast<const DW*>(ws[0]);
    HIPCHK(c, hipMemcpyAsync(act, xq, (size_t)nt * w0->mw.nb * sizeof(HyQ8K), hipMemcpyHostToDevice, c->s));
    size_t off = 0;
    for (int i = 0; i < cnt; i++) {
        const DW* w = reinterpret_cast<const DW*>(ws[i]);
        const bool direct = w->op_host && outs[i] == w->op_host && nt <= HY_MAX_BATCH;
        JobSpec j{w, direct ? w->op_dev : out + off, w->mw.n, EPI_STORE};
        MvOpts o;
        o.act = act;
        if (!run_multi(c, &j, 1, false, nt, o)) {
            c->broken = true;
            return false;
        }
        if (!direct) off += (size_t)w->mw.n * nt;
    }
    off = 0;
    for (int i = 0; i < cnt; i++) {
        const DW* w = reinterpret_cast<const DW*>(ws[i]);
        if (w->op_host && outs[i] == w->op_host && nt <= HY_MAX_BATCH) continue;
        const size_t nbytes = (size_t)w->mw.n * nt * sizeof(float);
        HIPCHK(c, hipMemcpyAsync(outs[i], out + off, nbytes, hipMemcpyDeviceToHost, c->s));
        off += (size_t)w->mw.n * nt;
    }
    HIPCHK(c, hipStreamSynchronize(c->s));
    return true;
}

// Per-op path (src/device.h:37-39; reference cu_matmul src/cuda.c:258-280): the weights of one
// group share the host's Q8_K activations; one synchronisation for the group. F16/F32 weights
// are rejected: the reference multiplies them with fp32 activations (src/kernels.c:1279-1300),
// which this entry point does not receive.
// Checks one per-op group; returns the bytes of its device staging (activations, then the
// outputs that are not written to weight_out buffers), or 0 when the group is refused.
static size_t matmul_staging(Ctx* c, hy_dweight* const* ws, float* const* outs, int cnt, const hymt2_q8k_block* xq,
                             int nt, size_t* act_bytes) {
    if (!c || c->broken || !ws || !outs || cnt < 1 || nt < 1 || nt > HY_MAX_CHUNK || !xq) return 0;
    const DW* w0 = reinterpret_cast<const DW*>(ws[0]);
    if (!w0) return 0;
    const int nb = w0->mw.nb;
    size_t out_total = 0;
    for (int i = 0; i < cnt; i++) {
        const DW* w = reinterpret_cast<const DW*>(ws[i]);
        if (!w || !outs[i] || w->mw.nb != nb || w->mw.k != w0->mw.k || !quant_kind(w->mw.kind)) {
            set_err(c, "matmul: weight %d unsupported for the per-op path", i);
            return 0;
        }
        if (!(w->op_host && outs[i] == w->op_host && nt <= HY_MAX_BATCH)) out_total += (size_t)w->mw.n * nt;
    }
    *act_bytes = ((size_t)nt * nb * sizeof(HyQ8K) + 255) / 256 * 256;
    return *act_bytes + out_total * sizeof(float);
}

static bool hip_matmul(void* impl, hy_dweight* const* ws, float* const* outs, int cnt, const hymt2_q8k_block* xq,
                       int nt) {
    Ctx* c = static_cast<Ctx*>(impl);
    size_t abytes = 0;
    const size_t total = matmul_staging(c, ws, outs, cnt, xq, nt, &abytes);
    if (!total || !ensure_scratch(c, abytes, total - abytes)) return false;
    return matmul_group(c, ws, outs, cnt, xq, nt, static_cast<HyQ8K*>(c->act), c->out);
}

// ----------------------------------------------------------------------------------- fused

// Drops the captured graphs. A device loop in progress replays g_step, so it ends here too
// (gen_steps then reports that no loop has begun).
static void free_graphs(Fused* f) {
    for (int v = 0; v < 2; v++) {
        if (f->g_fwd[v]) (void)hipGraphExecDestroy(f->g_fwd[v]);
        if (f->g_step[v]) (void)hipGraphExecDestroy(f->g_step[v]);
        if (f->g_steps[v]) (void)hipGraphExecDestroy(f->g_steps[v]);
        f->g_fwd[v] = f->g_step[v] = f->g_steps[v] = nullptr;
        f->sig_fwd[v].clear();
    }
    f->sig_step.clear();
    f->gen_total = 0;
}

static void free_fused(Fused* f) {
    if (!f) return;
    free_graphs(f);
    void* dev[] = {f->in_dev,  f->q,       f->k,       f->v,       f->ao,    f->g,       f->u,     f->logits,
                   f->act_h,   f->act_q,   f->act_f,   f->rope_c,  f->rope_s, f->out_norm, f->norms, f->kc,
                   f->vc,      f->slots,   f->ids,     f->sc,      f->segmax, f->p_h,     f->p_q,   f->p_k,
                   f->p_v,     f->p_ao,    f->p_g,     f->p_act_h, f->p_act_q, f->p_act_f};
    for (void* p : dev)
        if (p) (void)hipFree(p);
    if (f->in_host) (void)hipHostFree(f->in_host);
    if (f->stop) (void)hipFree(f->stop);
    if (f->stop_host) (void)hipHostFree(f->stop_host);
    delete f;
}

static bool same_shape(const Fused* f, const hymt2_fused_args* a) {
    return f && f->n_layer == a->n_layer && f->hidden == a->hidden && f->ffn == a->ffn && f->heads == a->heads &&
           f->kv_heads == a->kv_heads && f->hdim == a->hdim && f->qdim == a->qdim && f->kvdim == a->kvdim &&
           f->ctx == a->ctx && f->rope_half == a->rope_half;
}

// Allocates KV cache and work buffers for the model shape and copies norms and RoPE tables
// (reference cu_fused_prepare, src/cuda.c:282-337; idempotent for the same shape).
static bool copy_params(Ctx* c, const hymt2_fused_args* a) {
    Fused* f = c->f;
    const size_t H = f->hidden;
    const size_t rb = (size_t)a->ctx * a->rope_half * 4;
    HIPCHK(c, hipMemcpy(f->rope_c, a->rope_cos, rb, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(f->rope_s, a->rope_sin, rb, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(f->out_norm, a->out_norm, H * 4, hipMemcpyHostToDevice));
    for (int li = 0; li < a->n_layer; li++) {
        const hymt2_fused_layer& L = a->layers[li];
        HIPCHK(c, hipMemcpy(f->norm_ptr(li, 0), L.attn_norm, H * 4, hipMemcpyHostToDevice));
        HIPCHK(c, hipMemcpy(f->norm_ptr(li, 1), L.ffn_norm, H * 4, hipMemcpyHostToDevice));
        HIPCHK(c, hipMemcpy(f->norm_ptr(li, 2), L.q_norm, (size_t)a->hdim * 4, hipMemcpyHostToDevice));
        HIPCHK(c, hipMemcpy(f->norm_ptr(li, 3), L.k_norm, (size_t)a->hdim * 4, hipMemcpyHostToDevice));
    }
    if (f->eps != a->eps) free_graphs(f);  // captured kernels hold eps by value
    f->eps = a->eps;
    return true;
}

static bool hip_fused_prepare(void* impl, const hymt2_fused_args* a) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || !a || !a->layers) return false;
    // Same shape: keep the buffers and the KV cache (prefix reuse), refresh the parameters.
    if (same_shape(c->f, a)) return copy_params(c, a);
    if (a->hidden % 256 || a->ffn % 256 || a->qdim % 256 || a->heads % a->kv_heads || a->qdim != a->heads * a->hdim ||
        a->kvdim != a->kv_heads * a->hdim || (a->hdim != 64 && a->hdim != 128 && a->hdim != 256) ||
        2 * a->rope_half > a->hdim || a->ctx < 1 || (size_t)(a->ctx + 256) * 4 > 160 * 1024) {
        set_err(c, "fused_prepare: unsupported shape (hidden %d ffn %d qdim %d hdim %d ctx %d)", a->hidden, a->ffn,
                a->qdim, a->hdim, a->ctx);
        return false;
    }
    free_fused(c->f);
    c->f = nullptr;
    Fused* f = new Fused();
    f->n_layer = a->n_layer;
    f->hidden = a->hidden;
    f->ffn = a->ffn;
    f->heads = a->heads;
    f->kv_heads = a->kv_heads;
    f->hdim = a->hdim;
    f->qdim = a->qdim;
    f->kvdim = a->kvdim;
    f->ctx = a->ctx;
    f->rope_half = a->rope_half;
    f->eps = a->eps;
    const size_t B = HY_MAX_CHUNK, H = a->hidden, F = a->ffn, Q = a->qdim, KV = a->kvdim;
    f->in_bytes = kInH + B * H * 4;
    bool ok = dalloc(c, &f->in_dev, f->in_bytes) && hipHostMalloc(&f->in_host, f->in_bytes, 0) == hipSuccess;
    ok = ok && dalloc(c, &f->q, B * Q * 4) && dalloc(c, &f->k, B * KV * 4) && dalloc(c, &f->v, B * KV * 4) &&
         dalloc(c, &f->ao, B * Q * 4) && dalloc(c, &f->g, B * F * 4) && dalloc(c, &f->u, B * F * 4) &&
         dalloc(c, &f->act_h, B * (H / 256) * sizeof(HyQ8K)) && dalloc(c, &f->act_q, B * (Q / 256) * sizeof(HyQ8K)) &&
         dalloc(c, &f->act_f, B * (F / 256) * sizeof(HyQ8K)) &&
         dalloc(c, &f->rope_c, (size_t)a->ctx * a->rope_half * 4 + 4) &&
         dalloc(c, &f->rope_s, (size_t)a->ctx * a->rope_half * 4 + 4) && dalloc(c, &f->out_norm, H * 4) &&
         dalloc(c, &f->norms, (size_t)a->n_layer * (2 * H + 2 * a->hdim) * 4) &&
         dalloc(c, &f->kc, (size_t)a->n_layer * a->ctx * KV * 2) &&
         dalloc(c, &f->vc, (size_t)a->n_layer * a->ctx * KV * 2) && dalloc(c, &f->slots, (size_t)kArgSlots * 8) &&
         dalloc(c, &f->sc, (size_t)a->heads * split_sc_stride(a->ctx) * 4) &&
         dalloc(c, &f->segmax, (size_t)a->heads * split_seg_stride(a->ctx) * 4) &&
         dalloc(c, &f->stop, (kStopIds + 1) * sizeof(int));
    ok = ok && hipHostMalloc(&f->stop_host, 64, hipHostMallocMapped) == hipSuccess &&
         hipHostGetDevicePointer(reinterpret_cast<void**>(&f->stop_host_dev), f->stop_host, 0) == hipSuccess;
    if (!ok) {
        free_fused(f);
        return false;
    }
    f->d_pos = reinterpret_cast<int*>(f->in_dev);
    f->d_rope = reinterpret_cast<float*>(f->in_dev + 64);
    f->d_h = reinterpret_cast<float*>(f->in_dev + kInH);
    c->f = f;
    if (!copy_params(c, a)) return false;
    HIPCHK(c, hipMemset(f->kc, 0, (size_t)a->n_layer * a->ctx * KV * 2));
    HIPCHK(c, hipMemset(f->vc, 0, (size_t)a->n_layer * a->ctx * KV * 2));
    HIPCHK(c, hipMemset(f->slots, 0, (size_t)kArgSlots * 8));
    HIPCHK(c, hipMemset(f->in_dev, 0, f->in_bytes));
    return true;
}

// Stages pos and its RoPE row (cos[half], then sin[half]) at the front of in_host.
static void stage_pos(Fused* f, const hymt2_fused_args* a, int pos) {
    memcpy(f->in_host, &pos, 4);
    memcpy(f->in_host + 64, a->rope_cos + (size_t)pos * f->rope_half, (size_t)f->rope_half * 4);
    memcpy(f->in_host + 64 + (size_t)f->rope_half * 4, a->rope_sin + (size_t)pos * f->rope_half,
           (size_t)f->rope_half * 4);
}

static bool ensure_logits(Ctx* c, Fused* f, int n) {
    if ((size_t)n <= f->logits_cap) return true;
    if (f->logits) (void)hipFree(f->logits);
    f->logits = nullptr;
    f->logits_cap = 0;
    if (!dalloc(c, &f->logits, (size_t)n * 4)) return false;
    f->logits_cap = n;
    free_graphs(f);  // graphs hold the old pointer
    return true;
}

static const DW* dw(hy_dweight* p) { return reinterpret_cast<const DW*>(p); }

// Enqueues all layers of one forward of nt tokens (the order of src/model.c:822-886).
// nt == 1, per layer: [qkv matvec with the RMSNorm + Q8_K prologue] -> [attention block: RoPE,
// q/k norm, KV store, attention, Q8_K of the output] -> [o matvec + residual] -> [gate/up
// matvec with the RMSNorm prologue, SwiGLU and Q8_K epilogue] -> [down matvec + residual].
// nt > 1 quantizes each token's activations once into global memory and runs the general
// RoPE / attention kernels and the same matvec kernels over all tokens.
static bool enqueue_layers(Ctx* c, const hymt2_fused_args* a, int nt, int pos0, const int* pos_dev, bool split) {
    Fused* f = c->f;
    const int H = f->hidden, F = f->ffn, Q = f->qdim, KV = f->kvdim;
    for (int li = 0; li < f->n_layer; li++) {
        const hymt2_fused_layer& L = a->layers[li];
        const DW *wq = dw(L.wq), *wk = dw(L.wk), *wv = dw(L.wv), *wo = dw(L.wo), *wg = dw(L.wg), *wu = dw(L.wu),
                 *wd = dw(L.wd);
        if (!wq || !wk || !wv || !wo || !wg || !wu || !wd) {
            set_err(c, "fused_forward: layer %d has a missing device weight", li);
            return false;
        }
        const float* attn_norm = f->norm_ptr(li, 0);
        const float* ffn_norm = f->norm_ptr(li, 1);
        uint16_t* kc = f->kc + (size_t)li * f->ctx * KV;
        uint16_t* vc = f->vc + (size_t)li * f->ctx * KV;
        // ---- attention block
        JobSpec qkv[3] = {{wq, f->q, Q, EPI_STORE}, {wk, f->k, KV, EPI_STORE}, {wv, f->v, KV, EPI_STORE}};
        MvOpts o1;
        if (nt == 1) {
            o1.pro = PRO_NORM;
            o1.threads = 1024;
            o1.x = f->d_h;
            o1.norm_w = attn_norm;
            o1.eps = f->eps;
        } else {
            HIPCHK(c, launch_rmsnorm_q8k(f->d_h, attn_norm, f->eps, H, nt, nullptr, f->act_h, c->s));
            o1.act = f->act_h;
        }
        // single token: one workgroup per head (k_attn1) or, for long rows, the split form
        // (split_at), both with an fp32 output row that the o matvec quantizes; chunks: the
        // RoPE / KV-store kernel, then the chunk attention
        const bool head_attn = nt == 1;
        Attn1Args aa{};
        if (head_attn) {
            aa.q = f->q;
            aa.k = f->k;
            aa.v = f->v;
            aa.kc = kc;
            aa.vc = vc;
            aa.q_norm = f->norm_ptr(li, 2);
            aa.k_norm = f->norm_ptr(li, 3);
            aa.rope_cos = f->rope_c;
            aa.rope_sin = f->rope_s;
            aa.pos_dev = pos_dev;
            aa.rope_cur = pos_dev ? f->d_rope : nullptr;
            aa.pos0 = pos0;
            aa.ao = f->ao;
            aa.heads = f->heads;
            aa.kv_heads = f->kv_heads;
            aa.hdim = f->hdim;
            aa.rope_half = f->rope_half;
            aa.ctx = f->ctx;
            aa.eps = f->eps;
            aa.sc = f->sc;
            aa.segmax = f->segmax;
            aa.sc_stride = split_sc_stride(f->ctx);
            aa.seg_stride = split_seg_stride(f->ctx);
        }
        if (!(nt == 1 ? run_mv1(c, qkv, 3, false, o1) : run_multi(c, qkv, 3, false, nt, o1))) return false;
        if (head_attn) {
            HIPCHK(c, split ? launch_attn_split(aa, c->s) : launch_attn1(aa, c->s));
        } else {
            AttnArgs at{};
            at.q = f->q;
            at.k = f->k;
            at.v = f->v;
            at.kc = kc;
            at.vc = vc;
            at.ao = f->ao;
            at.q_norm = f->norm_ptr(li, 2);
            at.k_norm = f->norm_ptr(li, 3);
            at.rope_cos = f->rope_c;
            at.rope_sin = f->rope_s;
            at.pos_dev = pos_dev;
            at.pos0 = pos0;
            at.nt = nt;
            at.heads = f->heads;
            at.kv_heads = f->kv_heads;
            at.hdim = f->hdim;
            at.rope_half = f->rope_half;
            at.ctx = f->ctx;
            at.eps = f->eps;
            const bool fused_q = attention_quantizes(at);
            if (fused_q) at.act_out = f->act_q;
            HIPCHK(c, launch_rope_norm_store(at, c->s));
            HIPCHK(c, launch_attention(at, c->s));
            if (!fused_q) HIPCHK(c, launch_quantize_q8k(f->ao, Q, f->act_q, Q, nt, c->s));
        }
        JobSpec o{wo, f->d_h, H, EPI_ADD};
        MvOpts o2;
        o2.act = f->act_q;
        if (head_attn) {  // quantize the fp32 attention output in the matvec prologue
            o2.pro = PRO_QUANT;
            o2.threads = 1024;
            o2.x = f->ao;
            o2.act = nullptr;
        }
        if (!(nt == 1 ? run_mv1(c, &o, 1, false, o2) : run_multi(c, &o, 1, false, nt, o2))) return false;
        // ---- feed-forward block
        const bool pair = wg->mw.kind == wu->mw.kind && wg->mw.n == wu->mw.n;
        JobSpec gu[2] = {{wg, f->g, F, EPI_STORE}, {wu, f->u, F, EPI_STORE}};
        MvOpts o3;
        if (nt == 1) {
            o3.pro = PRO_NORM;
            o3.threads = 1024;
            o3.x = f->d_h;
            o3.norm_w = ffn_norm;
            o3.eps = f->eps;
        } else {
            HIPCHK(c, launch_rmsnorm_q8k(f->d_h, ffn_norm, f->eps, H, nt, nullptr, f->act_h, c->s));
            o3.act = f->act_h;
        }
        if (!(nt == 1 ? run_mv1(c, gu, 2, pair, o3) : run_multi(c, gu, 2, pair, nt, o3))) return false;
        if (!pair) HIPCHK(c, launch_silu_mul(f->g, f->u, nt * F, c->s));
        JobSpec dn{wd, f->d_h, H, EPI_ADD};
        MvOpts o4;
        if (nt == 1) {
            o4.pro = PRO_QUANT;
            o4.threads = 1024;
            o4.x = f->g;
        } else {
            HIPCHK(c, launch_quantize_q8k(f->g, F, f->act_f, F, nt, c->s));
            o4.act = f->act_f;
        }
        if (!(nt == 1 ? run_mv1(c, &dn, 1, false, o4) : run_multi(c, &dn, 1, false, nt, o4))) return false;
    }
    return true;
}

// Output RMSNorm + LM head on the last token (src/model.c:887-900), optionally folding the
// greedy argmax into f->slots (one key per workgroup of the head kernel; f->head_slots of them).
// Quantized heads run on the decode matvec over the Q8_K of the normalized last token.
static bool enqueue_head(Ctx* c, const hymt2_fused_args* a, int nt, bool argmax, int vocab_out,
                         const float* h_last = nullptr) {
    Fused* f = c->f;
    const DW* ow = dw(a->outw);
    if (!ow || ow->mw.k != f->hidden) {
        set_err(c, "fused_forward: missing or mismatched output weight");
        return false;
    }
    if (!ensure_logits(c, f, ow->mw.n)) return false;
    const float* hl = h_last ? h_last : f->d_h + (size_t)(nt - 1) * f->hidden;
    if (ow->mw.kind == KIND_F16 || ow->mw.kind == KIND_F32 || ow->mw.kind == KIND_Q8_0) {
        HeadArgs h{};
        h.W = ow->mw;
        h.h = hl;
        h.norm_w = f->out_norm;
        h.eps = f->eps;
        h.logits = f->logits;
        h.slots = argmax ? f->slots : nullptr;
        h.n_arg = vocab_out;
        if (argmax && head_grid(ow->mw.n) > kArgSlots) {
            set_err(c, "fused_forward: %d head rows exceed the argmax slots", ow->mw.n);
            return false;
        }
        HIPCHK(c, launch_head(h, c->s));
        f->head_slots = head_grid(ow->mw.n);
    } else {
        Mv1Launch L;
        memset(&L, 0, sizeof L);
        L.njobs = 1;
        L.job[0].W = ow->mw;
        L.job[0].out = f->logits;
        L.job[0].epi = EPI_STORE;
        L.act = f->act_h;
        L.slots = argmax ? f->slots : nullptr;
        L.n_arg = vocab_out;
        // RMSNorm + Q8_K of the last token once, not in every workgroup of the wide head grid
        HIPCHK(c, launch_rmsnorm_q8k(hl, f->out_norm, f->eps, f->hidden, 1, nullptr, f->act_h, c->s));
        const hipError_t e = launch_mv1(L, PRO_NONE, c->s);
        if (e == hipSuccess) {
            f->head_slots = L.grid;
        } else if (e != hipErrorNotSupported) {
            HIPCHK(c, e);
        } else {
            JobSpec j{ow, f->logits, ow->mw.n, EPI_STORE};
            MvOpts o;
            o.pro = PRO_NORM;
            o.x = hl;
            o.norm_w = f->out_norm;
            o.eps = f->eps;
            if (!run_matvec(c, &j, 1, false, 1, o)) return false;
            if (argmax) {
                if (argmax_grid(vocab_out) > kArgSlots) {
                    set_err(c, "fused_forward: vocab %d exceeds the argmax slots", vocab_out);
                    return false;
                }
                HIPCHK(c, launch_argmax(f->logits, vocab_out, f->slots, c->s));
                f->head_slots = argmax_grid(vocab_out);
            }
        }
    }
    return true;
}

static std::vector<const void*> weight_sig(const hymt2_fused_args* a) {
    std::vector<const void*> s;
    for (int li = 0; li < a->n_layer; li++) {
        const hymt2_fused_layer& L = a->layers[li];
        for (const void* p : {L.wq, L.wk, L.wv, L.wo, L.wg, L.wu, L.wd}) s.push_back(p);
    }
    s.push_back(a->outw);
    return s;
}

template <typename Fn>
static bool capture(Ctx* c, hipGraphExec_t* exec, Fn&& body) {
    hipGraph_t g = nullptr;
    HIPCHK(c, hipStreamBeginCapture(c->s, hipStreamCaptureModeThreadLocal));
    const bool ok = body();
    hipError_t e = hipStreamEndCapture(c->s, &g);
    if (!ok || e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        if (ok) set_err(c, "graph capture failed: %s", hipGetErrorString(e));
        return false;
    }
    e = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        set_err(c, "graph instantiate failed: %s", hipGetErrorString(e));
        return false;
    }
    return true;
}

// One forward of a->nt tokens at a->pos0 (reference cu_fused_forward, src/cuda.c:339-421):
// host h in, logits out when want_logits, KV written at absolute positions; exactly one host
// synchronisation. Single-token forwards replay a captured graph that reads pos0 from device
// memory, uploaded together with h in one copy.
static bool hip_fused_forward(void* impl, hymt2_fused_args* a) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || !a || !c->f || !same_shape(c->f, a) || a->nt < 1 || a->nt > HY_MAX_CHUNK || !a->h ||
        a->pos0 < 0 || a->pos0 + a->nt > c->f->ctx)
        return false;
    Fused* f = c->f;
    f->cache_n = 0;  // this forward writes K/V the device loop's prefix record does not know
    const int nt = a->nt;
    const size_t hbytes = (size_t)nt * f->hidden * 4;
    const bool logits = a->want_logits && a->outw && a->logits;
    memcpy(f->in_host + kInH, a->h, hbytes);
    if (nt == 1) {
        stage_pos(f, a, a->pos0);
        HIPCHK(c, hipMemcpyAsync(f->in_dev, f->in_host, kInH + hbytes, hipMemcpyHostToDevice, c->s));
        if (logits && !ensure_logits(c, f, dw(a->outw)->mw.n)) return false;
        std::vector<const void*> sig = weight_sig(a);
        sig.push_back(reinterpret_cast<const void*>((uintptr_t)logits));
        const int v = split_at(c, f, a->pos0) ? 1 : 0;
        if (!f->g_fwd[v] || f->sig_fwd[v] != sig) {
            if (f->g_fwd[v]) (void)hipGraphExecDestroy(f->g_fwd[v]);
            f->g_fwd[v] = nullptr;
            if (!capture(c, &f->g_fwd[v], [&] {
                    return enqueue_layers(c, a, 1, 0, f->d_pos, v == 1) && (!logits || enqueue_head(c, a, 1, false, 0));
                })) {
                c->broken = true;
                return false;
            }
            f->sig_fwd[v] = sig;
        }
        HIPCHK(c, hipGraphLaunch(f->g_fwd[v], c->s));
    } else {
        HIPCHK(c, hipMemcpyAsync(f->d_h, f->in_host + kInH, hbytes, hipMemcpyHostToDevice, c->s));
        if (!enqueue_layers(c, a, nt, a->pos0, nullptr, false) || (logits && !enqueue_head(c, a, nt, false, 0))) {
            c->broken = true;
            return false;
        }
    }
    if (logits) {
        HIPCHK(c, hipMemcpyAsync(a->logits, f->logits, (size_t)dw(a->outw)->mw.n * 4, hipMemcpyDeviceToHost, c->s));
    }
    HIPCHK(c, hipStreamSynchronize(c->s));
    return true;
}

// ----------------------------------------------------------------------------------- context

static void hip_destroy_impl(void* impl) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c) return;
    (void)hipSetDevice(c->dev);
    if (c->s) (void)hipStreamSynchronize(c->s);
    free_fused(c->f);
    if (c->act) (void)hipFree(c->act);
    if (c->out) (void)hipFree(c->out);
    for (hipEvent_t e : c->ev)
        if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : c->ring)
        if (e) (void)hipEventDestroy(e);
    if (c->s) (void)hipStreamDestroy(c->s);
    delete c;
}

static const hymt2_device_ops kOps = {hip_destroy_impl, hip_upload,        hip_release,       hip_matmul,
                                      hip_is_sw,        hip_weight_out,    hip_fused_prepare, hip_fused_forward};

extern "C" {

int hy_cuda_probe(char* out, int cap) {
    const int ok = access("/dev/kfd", R_OK | W_OK) == 0 ? 1 : 0;
    if (out && cap > 0) snprintf(out, (size_t)cap, "%d", ok);
    return ok;
}

void* hymt2_hip_open(char* info, size_t cap) {
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
        if (info && cap) snprintf(info, cap, "no HIP device");
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        if (info && cap) snprintf(info, cap, "hipSetDevice(0) failed");
        return nullptr;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (info && cap) snprintf(info, cap, "device 0 is %s; this build targets gfx950", prop.gcnArchName);
        return nullptr;
    }
    Ctx* c = new Ctx();
    c->dev = 0;
    if (hipStreamCreateWithFlags(&c->s, hipStreamNonBlocking) != hipSuccess) {
        if (info && cap) snprintf(info, cap, "hipStreamCreate failed");
        delete c;
        return nullptr;
    }
    for (hipEvent_t& e : c->ev) (void)hipEventCreate(&e);
    for (hipEvent_t& e : c->ring) (void)hipEventCreateWithFlags(&e, hipEventDisableTiming);
    c->scratch = scratch_address(c->dev);  // device 0 is current
    if (info && cap) snprintf(info, cap, "%s (%s, %d CUs)", prop.name[0] ? prop.name : "AMD GPU", prop.gcnArchName,
                              prop.multiProcessorCount);
    return c;
}

const hymt2_device_ops* hymt2_hip_ops(void) { return &kOps; }

hy_device* hy_cuda_create(const char* pref, char* info, size_t cap) {
    (void)pref;
    if (!hy_device_wrap) {
        if (info && cap) snprintf(info, cap, "hy_device_wrap not found: load through the hymt2 host library");
        return nullptr;
    }
    void* impl = hymt2_hip_open(info, cap);
    if (!impl) return nullptr;
    hy_device* d = hy_device_wrap(kDevKindCuda, "hip", impl, &kOps, false);
    if (!d) hip_destroy_impl(impl);
    return d;
}

int hymt2_hip_last_error(void* impl, char* out, int cap) {
    Ctx* c = static_cast<Ctx*>(impl);
    const char* s = c ? c->err.c_str() : "no context";
    if (out && cap > 0) snprintf(out, (size_t)cap, "%s", s);
    return (int)strlen(s);
}

int hymt2_hip_abi_layout(char* out, int cap) {
    return snprintf(out, (size_t)cap,
                    "weight_t=%zu weight_t.row_bytes=%zu weight_t.pk=%zu weight_t.gpu=%zu hy_fused_layer=%zu "
                    "hy_fused_args=%zu hy_fused_args.eps=%zu hy_fused_args.layers=%zu hy_fused_args.logits=%zu "
                    "hy_device_ops=%zu q8k_block=%zu",
                    sizeof(hymt2_weight), offsetof(hymt2_weight, row_bytes), offsetof(hymt2_weight, pk),
                    offsetof(hymt2_weight, gpu), sizeof(hymt2_fused_layer), sizeof(hymt2_fused_args),
                    offsetof(hymt2_fused_args, eps), offsetof(hymt2_fused_args, layers),
                    offsetof(hymt2_fused_args, logits), sizeof(hymt2_device_ops), sizeof(hymt2_q8k_block));
}

void* hymt2_hip_stream(void* impl) { return impl ? static_cast<Ctx*>(impl)->s : nullptr; }

int hymt2_hip_quantize_q8k(void* impl, const float* x, void* act, int k, int nt) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || k % 256 || nt < 1) return -1;
    return launch_quantize_q8k(x, k, static_cast<HyQ8K*>(act), k, nt, c->s) == hipSuccess ? 0 : -2;
}

int hymt2_hip_matvec(void* impl, hy_dweight* w, const void* act, float* out, int nt) {
    Ctx* c = static_cast<Ctx*>(impl);
    const DW* d = dw(w);
    if (!c || c->broken || !d || nt < 1 || nt > HY_MAX_CHUNK || !quant_kind(d->mw.kind)) return -1;
    JobSpec j{d, out, d->mw.n, EPI_STORE};
    MvOpts o;
    o.act = static_cast<const HyQ8K*>(act);
    return (nt == 1 ? run_mv1(c, &j, 1, false, o) : run_multi(c, &j, 1, false, nt, o)) ? 0 : -2;
}

int hymt2_hip_selftest_f16(void* impl, const uint16_t* src, float* dst, int n) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || n < 0) return -1;
    return launch_selftest(src, dst, n, 0, c->s) == hipSuccess ? 0 : -2;
}

int hymt2_hip_selftest_sqsum(void* impl, const float* x, int n, int m, float* out, int method) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || !x || !out) return -1;
    return launch_selftest_sqsum(x, n, m, out, method, c->s) == hipSuccess ? 0 : -2;
}

int hymt2_hip_selftest_mfma(void* impl, const float* a, const float* b, float* out, int nw) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || !a || !b || !out || nw < 1) return -1;
    return launch_selftest_mfma(a, b, out, nw, c->s) == hipSuccess ? 0 : -2;
}

int hymt2_hip_selftest_expf(void* impl, const float* src, float* dst, int n) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || n < 0) return -1;
    return launch_selftest(src, dst, n, 1, c->s) == hipSuccess ? 0 : -2;
}

int hymt2_hip_attn_split_from(void* impl, int from) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c) return -1;
    c->split_from = from < 0 ? kSplitFromDefault : from;
    if (c->f) free_graphs(c->f);
    return 0;
}

// Begins a device loop over positions 0 .. n_total - 1 whose first keep positions (keep <
// n_prompt) already hold the prompt's K/V; stop ids (at most kStopIds) are recorded by k_finish.
static int gen_begin_at(Ctx* c, const hymt2_fused_args* shape, hy_dweight* embd, int vocab_out, const int* prompt,
                        int n_prompt, int n_total, int keep, const int* stop_ids, int n_stop) {
    if (!c || c->broken || !shape || !prompt || n_prompt < 1 || n_total <= n_prompt || keep < 0 || keep >= n_prompt ||
        n_stop < 0 || n_stop > kStopIds || (n_stop && !stop_ids))
        return -1;
    if (!hip_fused_prepare(c, shape)) return -2;
    Fused* f = c->f;
    f->gen_total = 0;
    const DW* e = dw(embd);
    const DW* ow = dw(shape->outw);
    if (!e || !embed_kind(e->mw.kind) || e->mw.k != f->hidden || !ow) {
        set_err(c, "gen_begin: embedding must be an uploaded F16/F32/Q8_0/Q4_K/Q6_K [vocab][hidden] weight");
        return -3;
    }
    if (n_total > f->ctx || vocab_out < 1 || vocab_out > ow->mw.n || vocab_out > e->mw.n) {
        set_err(c, "gen_begin: %d positions exceed ctx %d (or bad vocab_out)", n_total, f->ctx);
        return -4;
    }
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= e->mw.n) {
            set_err(c, "gen_begin: prompt id %d out of range", prompt[i]);
            return -5;
        }
    if (n_total > f->ids_cap) {
        if (f->ids) (void)hipFree(f->ids);
        f->ids = nullptr;
        f->ids_cap = 0;
        if (!dalloc(c, &f->ids, (size_t)n_total * 4)) return -6;
        f->ids_cap = n_total;
        free_graphs(f);
    }
    if (!ensure_logits(c, f, ow->mw.n)) return -6;
    std::vector<const void*> sig = weight_sig(shape);
    sig.push_back(embd);
    sig.push_back(reinterpret_cast<const void*>((intptr_t)vocab_out));
    sig.push_back(reinterpret_cast<const void*>((intptr_t)n_prompt));
    sig.push_back(reinterpret_cast<const void*>((intptr_t)n_total));
    // the step graphs this loop's positions 0 .. n_total - 2 need (a step at position p replays
    // g_step[split_at(p)])
    const bool need[2] = {!split_at(c, f, 0), split_at(c, f, n_total - 2)};
    if (f->sig_step != sig || (need[0] && !f->g_step[0]) || (need[1] && !f->g_step[1])) {
        for (int v = 0; v < 2; v++) {
            if (f->g_step[v]) (void)hipGraphExecDestroy(f->g_step[v]);
            if (f->g_steps[v]) (void)hipGraphExecDestroy(f->g_steps[v]);
            f->g_step[v] = f->g_steps[v] = nullptr;
        }
        f->sig_step.clear();
        auto one_step = [&](int v) {
            if (!enqueue_layers(c, shape, 1, 0, f->d_pos, v == 1) || !enqueue_head(c, shape, 1, true, vocab_out))
                return false;
            const FinishArgs fa{f->slots,  f->head_slots, f->ids,    f->d_pos,     n_prompt, e->mw,
                                f->d_h,    f->hidden,     n_total,   f->rope_c,    f->rope_s, f->d_rope,
                                f->rope_half, f->ctx,     f->stop,   f->stop_host_dev};
            return launch_finish(fa, c->s) == hipSuccess;
        };
        for (int v = 0; v < 2; v++) {
            if (!need[v]) continue;
            if (!capture(c, &f->g_step[v], [&] { return one_step(v); })) return -7;
            if (!capture(c, &f->g_steps[v], [&] {
                    for (int i = 0; i < kStepsPerGraph; i++)
                        if (!one_step(v)) return false;
                    return true;
                }))
                return -7;
        }
        f->sig_step = sig;
    }
    // start state: ids[0..n_prompt) = prompt, pos = keep, h = embedding of ids[keep]; the stop
    // ids (-1 pads: no argmax equals it) and no stop yet
    int stv[kStopIds + 1];
    for (int j = 0; j < kStopIds; j++) stv[j] = j < n_stop ? stop_ids[j] : -1;
    stv[kStopIds] = INT_MAX;
    *f->stop_host = INT_MAX;
    memset(f->in_host, 0, f->in_bytes);
    stage_pos(f, shape, keep);
    if (hipMemcpyAsync(f->ids, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice, c->s) != hipSuccess ||
        hipMemcpyAsync(f->stop, stv, sizeof stv, hipMemcpyHostToDevice, c->s) != hipSuccess ||
        hipMemcpyAsync(f->in_dev, f->in_host, kInH, hipMemcpyHostToDevice, c->s) != hipSuccess ||
        launch_embed(f->ids, f->d_pos, e->mw, f->d_h, f->hidden, c->s) != hipSuccess ||
        hipStreamSynchronize(c->s) != hipSuccess) {
        set_err(c, "gen_begin: device setup failed");
        c->broken = true;
        return -8;
    }
    f->gen_total = n_total;
    f->gen_steps = keep;
    f->gen_keep = keep;
    f->gen_prompt = n_prompt;
    f->gen_vocab = vocab_out;
    f->gen_embd = e->mw;
    return 0;
}

int hymt2_hip_gen_begin(void* impl, const hymt2_fused_args* shape, hy_dweight* embd, int vocab_out,
                        const int* prompt, int n_prompt, int n_total) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (c && c->f) c->f->cache_n = 0;  // a loop the prefix record does not follow
    return gen_begin_at(c, shape, embd, vocab_out, prompt, n_prompt, n_total, 0, nullptr, 0);
}

// Whether the pipelined prefill applies: panel weights of the model's shapes in every layer
// (the GEMM), gate and up pairable, hidden 2048 (its RMSNorm kernel) and the chunk attention
// kernel with its fused Q8_K output.
static bool pipe_supported(const Fused* f, const hymt2_fused_args* a) {
    if (f->hidden != 2048) return false;
    AttnArgs at{};
    at.heads = f->heads;
    at.kv_heads = f->kv_heads;
    at.hdim = f->hdim;
    at.ctx = f->ctx;
    if (!attention_quantizes(at)) return false;
    auto panel = [](const DW* w, int n, int k) { return w && w->mw.kind == KIND_PANEL && w->mw.n == n && w->mw.k == k; };
    for (int li = 0; li < a->n_layer; li++) {
        const hymt2_fused_layer& L = a->layers[li];
        const int H = f->hidden, F = f->ffn, Q = f->qdim, KV = f->kvdim;
        if (!panel(dw(L.wq), Q, H) || !panel(dw(L.wk), KV, H) || !panel(dw(L.wv), KV, H) || !panel(dw(L.wo), H, Q) ||
            !panel(dw(L.wg), F, H) || !panel(dw(L.wu), F, H) || !panel(dw(L.wd), H, F))
            return false;
    }
    return true;
}

static bool ensure_pipe(Ctx* c, Fused* f) {
    if (f->p_h) return true;
    const size_t R = (size_t)kPipeMax * HY_MAX_CHUNK, H = f->hidden, F = f->ffn, Q = f->qdim, KV = f->kvdim;
    return dalloc(c, &f->p_h, R * H * 4) && dalloc(c, &f->p_q, R * Q * 4) && dalloc(c, &f->p_k, R * KV * 4) &&
           dalloc(c, &f->p_v, R * KV * 4) && dalloc(c, &f->p_ao, R * Q * 4) && dalloc(c, &f->p_g, R * F * 4) &&
           dalloc(c, &f->p_act_h, R * (H / 256) * sizeof(HyQ8K)) && dalloc(c, &f->p_act_q, R * (Q / 256) * sizeof(HyQ8K)) &&
           dalloc(c, &f->p_act_f, R * (F / 256) * sizeof(HyQ8K));
}

// The prompt of the device loop in chunks, pipelined over the layers: within a group of up to
// pipe_depth chunks (slot i = chunk g0 + i), launch step st runs layer st - i of every chunk i
// with 0 <= st - i < n_layer, each kernel of the layer once for all of them. Chunk i at layer l
// needs its own layer l - 1 (step st - 1) and the K/V that chunks before it stored at layer l
// (chunk i - 1 at step st - 1), so every chunk is the same forward over the same cache as in
// the one-after-another order, and the results are the same bits. Leaves the last token's
// hidden state in its slot for the head.
static bool enqueue_prefill_pipe(Ctx* c, const hymt2_fused_args* a, int chunk, const float** h_last) {
    Fused* f = c->f;
    const int np = f->gen_prompt, nl = f->n_layer, depth = c->pipe_depth, p0 = f->gen_keep;
    const int nc = (np - p0 + chunk - 1) / chunk;  // chunks of positions p0 .. np - 1
    const int H = f->hidden, F = f->ffn, Q = f->qdim, KV = f->kvdim;
    const size_t B = HY_MAX_CHUNK;
    for (int g0 = 0; g0 < nc; g0 += depth) {
        const int m = std::min(depth, nc - g0);
        auto tokens = [&](int i) { return std::min(chunk, np - p0 - (g0 + i) * chunk); };
        for (int i = 0; i < m; i++)
            HIPCHK(c, launch_embed_rows(f->ids, p0 + (g0 + i) * chunk, tokens(i), f->gen_embd, f->p_h + i * B * H, H,
                                        c->s));
        for (int st = 0; st < m + nl - 1; st++) {
            const int i0 = std::max(0, st - nl + 1), i1 = std::min(m - 1, st);
            const int nj = i1 - i0 + 1;
            PipeNorm n1{}, n2{};
            PipeAttn pa{};
            PipeQuant pq{};
            GemmPipeLaunch gq{}, go{}, gu{}, gd{};
            int rows = 0;
            for (int j = 0; j < nj; j++) {
                const int i = i0 + j, li = st - i, nt = tokens(i);
                const hymt2_fused_layer& L = a->layers[li];
                float* h = f->p_h + i * B * H;
                float* q = f->p_q + i * B * Q;
                float* k = f->p_k + i * B * KV;
                float* v = f->p_v + i * B * KV;
                float* g = f->p_g + i * B * F;
                HyQ8K* ah = f->p_act_h + i * B * (H / 256);
                HyQ8K* aq = f->p_act_q + i * B * (Q / 256);
                HyQ8K* af = f->p_act_f + i * B * (F / 256);
                n1.h[j] = n2.h[j] = h;
                n1.w[j] = f->norm_ptr(li, 0);
                n2.w[j] = f->norm_ptr(li, 1);
                n1.act[j] = n2.act[j] = ah;
                n1.row0[j] = n2.row0[j] = pa.row0[j] = pq.row0[j] = rows;
                auto job = [&](GemmPipeLaunch& G, hy_dweight* w, float* out, int ldo, int epi, const HyQ8K* act) {
                    GemmJob& J = G.job[G.njobs++];
                    J.W = dw(w)->mw;
                    J.out = out;
                    J.ldo = ldo;
                    J.epi = epi;
                    J.act = act;
                    J.nt = nt;
                };
                job(gq, L.wq, q, Q, EPI_STORE, ah);
                job(gq, L.wk, k, KV, EPI_STORE, ah);
                job(gq, L.wv, v, KV, EPI_STORE, ah);
                job(go, L.wo, h, H, EPI_ADD, aq);
                job(gu, L.wg, g, F, EPI_STORE, ah);  // pair: silu(gate) * up into g
                job(gu, L.wu, g, F, EPI_STORE, ah);
                job(gd, L.wd, h, H, EPI_ADD, af);
                AttnArgs& at = pa.a[j];
                at.q = q;
                at.k = k;
                at.v = v;
                at.kc = f->kc + (size_t)li * f->ctx * KV;
                at.vc = f->vc + (size_t)li * f->ctx * KV;
                at.ao = f->p_ao + i * B * Q;
                at.q_norm = f->norm_ptr(li, 2);
                at.k_norm = f->norm_ptr(li, 3);
                at.rope_cos = f->rope_c;
                at.rope_sin = f->rope_s;
                at.pos0 = p0 + (g0 + i) * chunk;
                at.nt = nt;
                at.heads = f->heads;
                at.kv_heads = f->kv_heads;
                at.hdim = f->hdim;
                at.rope_half = f->rope_half;
                at.ctx = f->ctx;
                at.eps = f->eps;
                at.act_out = aq;
                pq.x[j] = g;
                pq.act[j] = af;
                rows += nt;
            }
            n1.njobs = n2.njobs = pa.njobs = pq.njobs = nj;
            n1.eps = n2.eps = f->eps;
            pq.ldx = F;
            pq.K = F;
            gu.pair = 1;
            HIPCHK(c, launch_rmsnorm_q8k(n1, rows, c->s));
            HIPCHK(c, launch_gemm_panel(gq, c->s));
            HIPCHK(c, launch_rope_norm_store(pa, rows, c->s));
            HIPCHK(c, launch_attention(pa, rows, c->s));
            HIPCHK(c, launch_gemm_panel(go, c->s));
            HIPCHK(c, launch_rmsnorm_q8k(n2, rows, c->s));
            HIPCHK(c, launch_gemm_panel(gu, c->s));
            HIPCHK(c, launch_quantize_q8k(pq, rows, c->s));
            HIPCHK(c, launch_gemm_panel(gd, c->s));
        }
        if (g0 + m == nc) *h_last = f->p_h + (m - 1) * B * H + (size_t)(tokens(m - 1) - 1) * H;
    }
    return true;
}

int hymt2_hip_prefill_pipeline(void* impl, int depth) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c) return -1;
    const int prev = c->pipe_depth;
    if (depth >= 1) c->pipe_depth = std::min(depth, kPipeMax);
    return prev;
}

int hymt2_hip_gen_prefill(void* impl, const hymt2_fused_args* shape, int chunk) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || !c->f || !c->f->gen_total || !shape || !shape->layers) return -1;
    Fused* f = c->f;
    if (f->gen_steps != f->gen_keep || chunk < 1 || chunk > HY_MAX_CHUNK || !same_shape(f, shape)) {
        set_err(c, "gen_prefill: needs a fresh loop of the same shape and 1 <= chunk <= %d", HY_MAX_CHUNK);
        return -2;
    }
    const std::vector<const void*> sig = weight_sig(shape);
    if (f->sig_step.size() < sig.size() || !std::equal(sig.begin(), sig.end(), f->sig_step.begin())) {
        set_err(c, "gen_prefill: weights differ from the ones gen_begin captured");
        return -2;
    }
    const int np = f->gen_prompt, p0 = f->gen_keep;
    if (chunk > 1 && np - p0 > chunk && c->pipe_depth > 1 && pipe_supported(f, shape)) {
        const float* h_last = nullptr;
        if (!ensure_pipe(c, f) || !enqueue_prefill_pipe(c, shape, chunk, &h_last) ||
            !enqueue_head(c, shape, 1, true, f->gen_vocab, h_last)) {
            c->broken = true;
            return -3;
        }
    } else {
        for (int i = p0; i < np; i += chunk) {
            const int nt = std::min(chunk, np - i);
            if (launch_embed_rows(f->ids, i, nt, f->gen_embd, f->d_h, f->hidden, c->s) != hipSuccess ||
                !enqueue_layers(c, shape, nt, i, nullptr, nt == 1 && split_at(c, f, i)) ||
                (i + nt == np && !enqueue_head(c, shape, nt, true, f->gen_vocab))) {
                c->broken = true;
                return -3;
            }
        }
    }
    // position np - 1 has been processed: the finishing kernel records the first generated id,
    // embeds it and advances the step counter to np, where the step graph continues
    const FinishArgs fa{f->slots,  f->head_slots, f->ids,       f->d_pos,  np,       f->gen_embd,
                        f->d_h,    f->hidden,     f->gen_total, f->rope_c, f->rope_s, f->d_rope,
                        f->rope_half, f->ctx,     f->stop,      f->stop_host_dev};
    if (launch_set_int(f->d_pos, np - 1, c->s) != hipSuccess || launch_finish(fa, c->s) != hipSuccess) {
        set_err(c, "gen_prefill: launch failed");
        c->broken = true;
        return -3;
    }
    f->gen_steps = np;
    return 0;
}

int hymt2_hip_gen_steps(void* impl, int n) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || !c->f || !c->f->gen_total || n < 0) return -1;
    Fused* f = c->f;
    if (f->gen_steps + n > f->gen_total - 1) {
        set_err(c, "gen_steps: %d + %d steps exceed the %d positions of this loop", f->gen_steps, n, f->gen_total);
        return -2;
    }
    // kStepsPerGraph steps per launch where their positions share one attention form, else one
    for (int i = 0; i < n;) {
        const int p = f->gen_steps + i;
        const int v = split_at(c, f, p) ? 1 : 0;
        const bool many = n - i >= kStepsPerGraph && (split_at(c, f, p + kStepsPerGraph - 1) ? 1 : 0) == v;
        if (hipGraphLaunch(many ? f->g_steps[v] : f->g_step[v], c->s) != hipSuccess) {
            set_err(c, "gen_steps: hipGraphLaunch failed");
            c->broken = true;
            return -3;
        }
        i += many ? kStepsPerGraph : 1;
    }
    f->gen_steps += n;
    return 0;
}

int hymt2_hip_gen_read(void* impl, int* ids, int first, int count) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || !c->f || !c->f->gen_total || !ids || first < 0 || count < 0 ||
        first + count > c->f->gen_total)
        return -1;
    if (hipMemcpyAsync(ids, c->f->ids + first, (size_t)count * 4, hipMemcpyDeviceToHost, c->s) != hipSuccess ||
        hipStreamSynchronize(c->s) != hipSuccess) {
        set_err(c, "gen_read: copy failed");
        c->broken = true;
        return -2;
    }
    return count;
}

int hymt2_hip_generate_chunked(void* impl, const hymt2_fused_args* shape, hy_dweight* embd, int vocab_out,
                               const int* prompt, int n_prompt, int n_gen, int chunk, int* out_ids,
                               hymt2_gen_stats* stats) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || !out_ids || n_gen < 1 || chunk < 1) return -1;
    if (c->f) c->f->cache_n = 0;  // a loop the prefix record does not follow
    int rc = gen_begin_at(c, shape, embd, vocab_out, prompt, n_prompt, n_prompt + n_gen, 0, nullptr, 0);
    if (rc) return rc;
    (void)hipEventRecord(c->ev[0], c->s);
    if ((rc = chunk > 1 ? hymt2_hip_gen_prefill(impl, shape, chunk) : hymt2_hip_gen_steps(impl, n_prompt))) return rc;
    (void)hipEventRecord(c->ev[1], c->s);
    if ((rc = hymt2_hip_gen_steps(impl, n_gen - 1))) return rc;
    (void)hipEventRecord(c->ev[2], c->s);
    if ((rc = hymt2_hip_gen_read(impl, out_ids, n_prompt, n_gen)) != n_gen) return rc;
    if (stats) {
        float a = 0.f, b = 0.f;
        (void)hipEventElapsedTime(&a, c->ev[0], c->ev[1]);
        (void)hipEventElapsedTime(&b, c->ev[1], c->ev[2]);
        stats->prefill_ms = a;
        stats->decode_ms = b;
        stats->prefill_steps = n_prompt;
        stats->decode_steps = n_gen - 1;
        stats->cached_tokens = 0;
    }
    return n_gen;
}

int hymt2_hip_generate(void* impl, const hymt2_fused_args* shape, hy_dweight* embd, int vocab_out, const int* prompt,
                       int n_prompt, int n_gen, int* out_ids, hymt2_gen_stats* stats) {
    return hymt2_hip_generate_chunked(impl, shape, embd, vocab_out, prompt, n_prompt, n_gen, 1, out_ids, stats);
}

// What the K/V of a device-loop sequence depends on besides its ids: the weights, the norms,
// the RoPE tables and eps (the shape is the Fused's own).
static std::vector<const void*> cache_sig(const hymt2_fused_args* a, const hy_dweight* embd) {
    std::vector<const void*> s = weight_sig(a);
    s.push_back(embd);
    s.push_back(a->rope_cos);
    s.push_back(a->rope_sin);
    for (int li = 0; li < a->n_layer; li++) {
        const hymt2_fused_layer& L = a->layers[li];
        for (const void* p : {(const void*)L.attn_norm, (const void*)L.ffn_norm, (const void*)L.q_norm,
                              (const void*)L.k_norm})
            s.push_back(p);
    }
    uint32_t eb;
    memcpy(&eb, &a->eps, 4);
    s.push_back(reinterpret_cast<const void*>((uintptr_t)eb));
    return s;
}

int hymt2_hip_generate_ids(void* impl, const hymt2_fused_args* shape, hy_dweight* embd, int vocab_out,
                           const int* prompt, int n_prompt, int max_tokens, const hymt2_gen_opts* opts,
                           int* out_ids, hymt2_gen_stats* stats) {
    Ctx* c = static_cast<Ctx*>(impl);
    if (!c || c->broken || !shape || !shape->layers || !prompt || n_prompt < 1 || !out_ids) return -1;
    const int chunk = opts && opts->chunk > 0 ? opts->chunk : 1;
    const int n_stop = opts ? opts->n_stop : 0;
    if (chunk > HY_MAX_CHUNK || n_stop < 0 || n_stop > kStopIds || (n_stop && !opts->stop_ids)) {
        set_err(c, "generate_ids: chunk must be 1..%d and at most %d stop ids", HY_MAX_CHUNK, kStopIds);
        return -1;
    }
    if (!hip_fused_prepare(impl, shape)) return -2;
    Fused* f = c->f;
    // max_tokens capped at the positions the context has left (src/model.c:925-926)
    if (n_prompt + max_tokens > f->ctx) max_tokens = f->ctx - n_prompt;
    if (max_tokens <= 0) {
        set_err(c, "generate_ids: a prompt of %d ids leaves no room in ctx %d", n_prompt, f->ctx);
        return -4;
    }
    // the K/V of the longest common prefix with the cached sequence, at most n - 1 positions
    // (src/model.c:930-936)
    const std::vector<const void*> sig = cache_sig(shape, embd);
    int keep = 0;
    if (opts && opts->reuse_prefix && f->cache_sig == sig)
        while (keep < f->cache_n && keep < n_prompt - 1 && f->cache_tok[keep] == prompt[keep]) keep++;
    f->cache_n = 0;  // until this loop has finished
    int rc = gen_begin_at(c, shape, embd, vocab_out, prompt, n_prompt, n_prompt + max_tokens, keep,
                          n_stop ? opts->stop_ids : nullptr, n_stop);
    if (rc) return rc;
    (void)hipEventRecord(c->ev[0], c->s);
    if ((rc = chunk > 1 ? hymt2_hip_gen_prefill(impl, shape, chunk) : hymt2_hip_gen_steps(impl, n_prompt - keep)))
        return rc;
    (void)hipEventRecord(c->ev[1], c->s);
    // decode steps in launches of kStepsPerGraph, at most two in flight: before a launch the host
    // waits for the one two launches back and reads the stop position, so the GPU always has the
    // next launch queued and at most two launches' steps run on past a stop (their K/V lies past
    // the sequence's end and their ids are not read)
    const int total = max_tokens - 1;
    int done = 0;
    for (int launch = 0; done < total; launch++) {
        if (launch >= 2) {
            if (hipEventSynchronize(c->ring[launch & 1]) != hipSuccess) {
                set_err(c, "generate_ids: event wait failed");
                c->broken = true;
                return -3;
            }
            if (*reinterpret_cast<volatile int*>(f->stop_host) != INT_MAX) break;
        }
        const int k = std::min(kStepsPerGraph, total - done);
        if ((rc = hymt2_hip_gen_steps(impl, k))) return rc;
        (void)hipEventRecord(c->ring[launch & 1], c->s);
        done += k;
    }
    (void)hipEventRecord(c->ev[2], c->s);
    int stop_at = INT_MAX;
    if (hipMemcpyAsync(&stop_at, f->stop + kStopIds, sizeof stop_at, hipMemcpyDeviceToHost, c->s) != hipSuccess ||
        hipStreamSynchronize(c->s) != hipSuccess) {
        set_err(c, "generate_ids: reading the stop position failed");
        c->broken = true;
        return -3;
    }
    // the ids before the stop id, or max_tokens of them (src/model.c:944-951)
    const bool stopped = stop_at != INT_MAX;
    const int ng = stopped ? stop_at - n_prompt : max_tokens;
    if (ng > 0 && (rc = hymt2_hip_gen_read(impl, out_ids, n_prompt, ng)) != ng) return rc < 0 ? rc : -3;
    // the cache holds the prompt and the ids fed back: all generated ids after a stop, all but
    // the last after a full run (src/model.c:948-953)
    const int fed = stopped ? ng : ng - 1;
    f->cache_tok.assign(prompt, prompt + n_prompt);
    f->cache_tok.insert(f->cache_tok.end(), out_ids, out_ids + fed);
    f->cache_n = n_prompt + fed;
    f->cache_sig = sig;
    if (stats) {
        float a = 0.f, b = 0.f;
        (void)hipEventElapsedTime(&a, c->ev[0], c->ev[1]);
        (void)hipEventElapsedTime(&b, c->ev[1], c->ev[2]);
        stats->prefill_ms = a;
        stats->decode_ms = b;
        stats->prefill_steps = n_prompt - keep;
        stats->decode_steps = done;
        stats->cached_tokens = keep;
    }
    return ng;
}

bool hymt2_hip_matmul_static(void* impl, hy_dweight* const* ws, float* const* outs, int cnt,
                             const hymt2_q8k_block* xq, int nt) {
    Ctx* c = static_cast<Ctx*>(impl);
    size_t abytes = 0;
    const size_t total = matmul_staging(c, ws, outs, cnt, xq, nt, &abytes);
    if (!total) return false;
    if (!c->scratch) {
        set_err(c, "matmul_static: the device address of the static scratch is unavailable");
        return false;
    }
    if (total > kScratchBytes) {
        set_err(c, "matmul_static: the group needs %zu bytes of staging, more than the %zu-byte static scratch", total,
                kScratchBytes);
        return false;
    }
    return matmul_group(c, ws, outs, cnt, xq, nt, reinterpret_cast<HyQ8K*>(c->scratch),
                        reinterpret_cast<float*>(c->scratch + abytes));
}

int hymt2_hip_head(void* impl, hy_dweight* w, const float* h, const float* norm_w, float eps, float* logits,
                   int n_arg, unsigned long long* key) {
    Ctx* c = static_cast<Ctx*>(impl);
    const DW* d = dw(w);
    if (!c || c->broken || !d || (d->mw.kind != KIND_F16 && d->mw.kind != KIND_F32 && d->mw.kind != KIND_Q8_0) ||
        n_arg > d->mw.n)
        return -1;
    HeadArgs a{};
    a.W = d->mw;
    a.h = h;
    a.norm_w = norm_w;
    a.eps = eps;
    a.logits = logits;
    a.argmax_key = key;
    a.n_arg = n_arg;
    return launch_head(a, c->s) == hipSuccess ? 0 : -2;
}

int hymt2_hip_ffn_in(void* impl, hy_dweight* wg, hy_dweight* wu, const float* h, const float* norm_w, float eps,
                     float* out) {
    Ctx* c = static_cast<Ctx*>(impl);
    const DW *g = dw(wg), *u = dw(wu);
    if (!c || c->broken || !g || !u || g->mw.kind != u->mw.kind || g->mw.n != u->mw.n || g->mw.k != u->mw.k ||
        !quant_kind(g->mw.kind) || !h || !norm_w || !out)
        return -1;
    JobSpec gu[2] = {{g, out, g->mw.n, EPI_STORE}, {u, out, u->mw.n, EPI_STORE}};
    MvOpts o;
    o.pro = PRO_NORM;
    o.threads = 1024;
    o.x = h;
    o.norm_w = norm_w;
    o.eps = eps;
    return run_mv1(c, gu, 2, true, o) ? 0 : -2;
}

}  // extern "C"
