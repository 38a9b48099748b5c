/* hymt2_hip.h: C ABI of the MI355X (gfx950) HIP backend for the Hy-MT2 token loop.
 *
 * libhymt2_hip.so plugs into the reference host (zhangbo8418/hymt2) exactly where its CUDA
 * backend does: the host's device layer calls hy_cuda_create / hy_cuda_probe as extern symbols
 * (src/device.c:8-9, :79, :168), so linking this library instead of src/cuda.c selects it with
 * HYMT2_DEVICE=cuda (or auto) and leaves model.c, device.c, gguf.c, tokenizer.c and hymt2.h
 * unchanged. The device it reports is named "hip".
 *
 * The structs below are byte-for-byte mirrors of the reference's interface types; the library
 * checks their sizes and offsets at compile time and reports them through
 * hymt2_hip_abi_layout() for the ABI tests.
 *
 * Numerics: every result equals the reference's scalar CPU path (HYMT2_ISA=scalar,
 * HYMT2_REPACK=1) bit for bit: int32 block dots, fp32 matvec outputs, norms, RoPE, attention,
 * SwiGLU, logits and greedy token ids.
 */
#ifndef HYMT2_HIP_H
#define HYMT2_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HYMT2_HIP_API __attribute__((visibility("default")))

/* Tokens per call that matmul and fused_forward accept. The reference host sends at most
 * MAX_BATCH = 16 (src/internal.h:12); a host built with MAX_BATCH up to 128 can send 128-token
 * prefill chunks, which run on the int8-MFMA GEMM. */
#define HYMT2_HIP_MAX_CHUNK 128

/* ---------------------------------------------------------------- reference ABI mirrors */

typedef struct hy_device hy_device;   /* opaque, owned by the host (src/device.c:18-24) */
typedef struct hy_dweight hy_dweight; /* opaque device weight, owned by this backend */

/* == weight_t, src/internal.h:48-61 (64 bytes on LP64) */
typedef struct hymt2_weight {
    const uint8_t *data;  /* raw GGUF rows */
    int type;             /* ggml type: 0 F32, 1 F16, 12 Q4_K, 14 Q6_K, 40 Q2_0C, 43 STQ1_0 */
    int k;                /* input dim */
    int n;                /* rows */
    size_t row_bytes;
    const uint8_t *pk;    /* panel codes n*(k/256)*64 B (STQ1_0 / Q2_0C) */
    const float *ps;      /* panel scales n*(k/256) */
    int pshift, poff;
    void *gpu;
} hymt2_weight;

/* == q8k_block, src/internal.h:29-41 (576 bytes, 64-byte aligned) */
typedef struct hymt2_q8k_block {
    int8_t qp[256];
    float d;
    int32_t sum;
    int16_t bsums[16];
    uint8_t pad[24];
    int8_t qs[256];
} hymt2_q8k_block;

/* == hy_fused_layer, src/device.h:44-47 */
typedef struct hymt2_fused_layer {
    hy_dweight *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
} hymt2_fused_layer;

/* == hy_fused_args, src/device.h:49-59 */
typedef struct hymt2_fused_args {
    int n_layer, hidden, ffn, heads, kv_heads, hdim, qdim, kvdim, ctx, rope_half, nt, pos0;
    float eps;
    int want_logits;
    hymt2_fused_layer *layers;
    hy_dweight *outw;
    const float *out_norm;
    const float *rope_cos, *rope_sin; /* [ctx * rope_half] */
    float *h;      /* in: [nt * hidden] after the host embedding */
    float *logits; /* out when want_logits: [outw->n] */
} hymt2_fused_args;

/* == hy_device_ops, src/device.h:70-80 */
typedef struct hymt2_device_ops {
    void (*destroy_impl)(void *impl);
    hy_dweight *(*upload)(void *impl, const hymt2_weight *w);
    void (*release)(hy_dweight *w);
    bool (*matmul)(void *impl, hy_dweight *const *ws, float *const *outs, int cnt, const hymt2_q8k_block *xq, int nt);
    bool (*is_software)(const void *impl);
    float *(*weight_out)(hy_dweight *w);
    bool (*fused_prepare)(void *impl, const hymt2_fused_args *shape);
    bool (*fused_forward)(void *impl, hymt2_fused_args *a);
} hymt2_device_ops;

/* ---------------------------------------------------------------- drop-in entry points */

/* Replaces hy_cuda_create, src/cuda.c:151-183. Creates the HIP context on device 0 and wraps
 * it with the host's hy_device_wrap (src/device.c:25-35) under the name "hip". Returns NULL
 * with a message in info when no gfx950 device is usable or when the library is loaded
 * without the reference host (hy_device_wrap absent). */
HYMT2_HIP_API hy_device *hy_cuda_create(const char *pref, char *info, size_t cap);

/* Replaces hy_cuda_probe, src/cuda.c:18-34: writes "1" when the amdgpu compute node /dev/kfd
 * is accessible, else "0"; returns the same as an int. Like the reference's probe (which only
 * dlopens the runtime), it never initialises the GPU. */
HYMT2_HIP_API int hy_cuda_probe(char *out, int cap);

/* ---------------------------------------------------------------- extensions (no counterpart
 * in the reference interface) */

/* The backend context and vtable without the reference host: the same impl pointer and
 * hy_device_ops table that hy_cuda_create hands to hy_device_wrap. For callers that drive the
 * backend directly (benchmarks, tests, FFI users without the C host). */
HYMT2_HIP_API void *hymt2_hip_open(char *info, size_t cap);
HYMT2_HIP_API const hymt2_device_ops *hymt2_hip_ops(void);

/* Last error message of a context ("" if none); returns its length. */
HYMT2_HIP_API int hymt2_hip_last_error(void *impl, char *out, int cap);

/* "name=value" list of the ABI struct sizes and offsets this library was compiled with. */
HYMT2_HIP_API int hymt2_hip_abi_layout(char *out, int cap);

/* The context's HIP stream (hipStream_t), on which every kernel of the context runs. */
HYMT2_HIP_API void *hymt2_hip_stream(void *impl);

/* Kernel-level entry points on device pointers, enqueued on the context stream (asynchronous;
 * 0 on success, negative on error):
 *   quantize_q8k: x[nt][k] fp32 -> act[nt][k/256] q8k_block (quantize_q8k, src/kernels.c:128)
 *   matvec:       out[t*n + r] = row r of an uploaded weight . act[t] (matmul_rows,
 *                 src/kernels.c:1241), panel / Q4_K / Q6_K weights, 1 <= nt <= 128; above 16
 *                 tokens panel weights run on the int8-MFMA GEMM */
HYMT2_HIP_API int hymt2_hip_quantize_q8k(void *impl, const float *x_dev, void *act_dev, int k, int nt);
HYMT2_HIP_API int hymt2_hip_matvec(void *impl, hy_dweight *w, const void *act_dev, float *out_dev, int nt);

/* The per-op matmul of the vtable (hy_device_ops.matmul, same arguments and results) with no
 * allocation: no counterpart in the reference interface. It is for callers that cannot
 * allocate device memory (hipMalloc) while they run: code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation. Its device staging (the Q8_K activations copied from
 * xq, then the outputs that go back by copy rather than into weight_out buffers) lives in one
 * static 16 MiB array per GPU, held until the process ends; a group that needs more staging is
 * refused (false, with a message). All calls on one GPU share that array, so calls that overlap
 * on one GPU race. It calls no hipMalloc / hipFree. */
HYMT2_HIP_API bool hymt2_hip_matmul_static(void *impl, hy_dweight *const *ws, float *const *outs, int cnt,
                                           const hymt2_q8k_block *xq, int nt);

/* Device self-checks of the scalar conversions the kernels use (same device functions):
 * f16 -> f32 and expf over n inputs. */
HYMT2_HIP_API int hymt2_hip_selftest_f16(void *impl, const uint16_t *src_dev, float *dst_dev, int n);
HYMT2_HIP_API int hymt2_hip_selftest_expf(void *impl, const float *src_dev, float *dst_dev, int n);
/* The RMSNorm sum of squares of m vectors x[m][n] (n <= 2048, n % 4 == 0): out[v] = the
 * sequential fp32 sum x0*x0 + x1*x1 + ... (src/model.c:719-739), by the lane-serial chain
 * (method 0), the one-wavefront exact segmented form (method 1) or the workgroup-wide exact
 * form of the decode matvec's RMSNorm (method 2). Method 3: the plain sequential sum
 * x0 + x1 + ... of n <= 4096 non-negative values by the 8-wavefront exact form of the decode
 * attention's softmax denominator (src/model.c:781-789). */
HYMT2_HIP_API int hymt2_hip_selftest_sqsum(void *impl, const float *x_dev, int n, int m, float *out_dev, int method);
/* The fp32 products of the four-token chunk attention's matrix-core form (no counterpart in the
 * reference: it checks an instruction property the attention's bit-exactness rests on):
 * v_mfma_f32_16x16x1f32 with a zero accumulator over nw wavefronts of 64 operand pairs
 * a[w][lane], b[w][lane]; out[w][r][lane] = a[w][16 (r/4) + 4 (lane/16) + r%4] *
 * b[w][16 (r/4) + lane%16], each the separately rounded fp32 product (a -0 product as +0). */
HYMT2_HIP_API int hymt2_hip_selftest_mfma(void *impl, const float *a_dev, const float *b_dev, float *out_dev, int nw);

/* Device-resident greedy generation (no host round trip per token). Each step runs one
 * position through the fused forward and the LM head; the argmax (first index on ties over
 * the first vocab_out rows, src/model.c:945-948) becomes the next step's token, whose
 * embedding row the device gathers itself. While the prompt lasts, its next id is used
 * instead. These entry points run a fixed number of steps from position 0 (stop ids and prefix
 * reuse: hymt2_hip_generate_ids below). `shape` is a hy_fused_args carrying layers, outw,
 * norms and RoPE tables (prepared on first use); `embd` is the uploaded F16/F32 token
 * embedding (the tied head weight is allowed).
 *   gen_begin: uploads the prompt, resets position/argmax state, embeds prompt[0]; n_total is
 *              the number of positions the loop may fill (<= ctx).
 *   gen_steps: enqueues n steps (asynchronous; replays of one captured graph); at most
 *              n_total - 1 steps in all.
 *   gen_read:  waits for the stream and copies ids[first .. first + count).
 *   gen_prefill: instead of the first n_prompt steps, runs the whole prompt as chunks of up to
 *              `chunk` (<= 128) positions through the multi-token forward (int8-MFMA GEMMs
 *              for panel weights, causal attention over the growing KV cache), then the LM
 *              head on the last prompt position; the loop continues with gen_steps exactly as
 *              after n_prompt steps (bit-identical ids, logits and KV cache). The prompt pass
 *              of the reference's gen_ids (src/model.c:928-937, forward_tokens :904-909).
 *   generate:  begin + n_prompt steps + (n_gen - 1) steps + read of the n_gen generated ids,
 *              with HIP-event timings of the two phases. Returns n_gen.
 *   generate_chunked: the same with the prompt through gen_prefill(chunk) (chunk 1: steps). */
typedef struct hymt2_gen_stats {
    double prefill_ms;  /* steps that consume prompt ids */
    double decode_ms;   /* steps that consume generated ids */
    int prefill_steps, decode_steps;
    int cached_tokens;  /* prompt positions whose K/V was reused (hymt2_hip_generate_ids) */
} hymt2_gen_stats;
HYMT2_HIP_API int hymt2_hip_gen_begin(void *impl, const hymt2_fused_args *shape, hy_dweight *embd, int vocab_out,
                                      const int *prompt, int n_prompt, int n_total);
HYMT2_HIP_API int hymt2_hip_gen_steps(void *impl, int n);
HYMT2_HIP_API int hymt2_hip_gen_prefill(void *impl, const hymt2_fused_args *shape, int chunk);
HYMT2_HIP_API int hymt2_hip_gen_read(void *impl, int *ids, int first, int count);
HYMT2_HIP_API int hymt2_hip_generate(void *impl, const hymt2_fused_args *shape, hy_dweight *embd, int vocab_out,
                                     const int *prompt, int n_prompt, int n_gen, int *out_ids,
                                     hymt2_gen_stats *stats);
HYMT2_HIP_API int hymt2_hip_generate_chunked(void *impl, const hymt2_fused_args *shape, hy_dweight *embd,
                                             int vocab_out, const int *prompt, int n_prompt, int n_gen, int chunk,
                                             int *out_ids, hymt2_gen_stats *stats);

/* The reference's greedy loop gen_ids (src/model.c:914-958) from the prompt ids on, on the
 * device (the chat template and the tokenizer stay with the host; src/model.c:915-923):
 *   - max_tokens is capped at ctx - n_prompt (src/model.c:925-926; nothing left: error);
 *   - with reuse_prefix, the K/V of the longest common prefix of the prompt and the sequence the
 *     previous hymt2_hip_generate_ids call left in the cache is kept, at most n_prompt - 1
 *     positions (src/model.c:930-936); only the same weights, norms, RoPE tables and eps reuse
 *     it, and any fused_forward or other device loop in between drops it;
 *   - the rest of the prompt runs in chunks of `chunk` positions (1: single-token steps);
 *   - then greedy ids (first index on ties) until one of stop_ids comes up, which ends the loop
 *     and is not returned (tok_is_stop, src/tokenizer.c:179: the model's eos and eog), or
 *     max_tokens ids. The device checks the ids itself; the host keeps at most two launches of
 *     8 steps in flight and stops launching after a stop (those steps' K/V lies past the end of
 *     the sequence and their ids are not read).
 * Returns the number of ids written to out_ids (>= 0), negative on errors (hymt2_hip_last_error).
 * stats (optional): prefill_steps = positions computed for the prompt, decode_steps = steps
 * run after it, cached_tokens = positions reused. No counterpart in the reference interface:
 * its loop calls fused_forward once per token and reads the logits back. */
typedef struct hymt2_gen_opts {
    const int *stop_ids; /* ids that end the loop (eos, eog); up to 8 */
    int n_stop;
    int chunk;           /* prompt positions per forward, 1 .. 128 (0: 1) */
    int reuse_prefix;    /* nonzero: reuse the K/V prefix as the reference's loop does */
} hymt2_gen_opts;
HYMT2_HIP_API int hymt2_hip_generate_ids(void *impl, const hymt2_fused_args *shape, hy_dweight *embd, int vocab_out,
                                         const int *prompt, int n_prompt, int max_tokens,
                                         const hymt2_gen_opts *opts, int *out_ids, hymt2_gen_stats *stats);

/* Single-token attention form by position (no counterpart in the reference interface): a forward
 * at position >= from (fused_forward with nt == 1, and the device loop's steps) runs the split
 * attention, whose scores use many CUs (k_attn_scores, then k_attn_out); positions below run
 * the one-workgroup-per-head kernel (k_attn1). Both give the same bits. from < 0 restores the
 * default. Shapes k_attn1 does not take (head dim other than 64/128, ctx > 4096) always split.
 * Drops the captured graphs (and ends a device loop in progress). 0 on success. */
HYMT2_HIP_API int hymt2_hip_attn_split_from(void *impl, int from);

/* Chunks in flight in hymt2_hip_gen_prefill (no counterpart in the reference interface; the
 * reference runs one chunk after another, src/model.c:914-958). With depth > 1 a prompt of
 * several chunks runs pipelined over the layers: chunk i's layer l in the same launches as
 * chunk i + 1's layer l - 1, up to depth chunks at a time. Every chunk is the same forward over
 * the same KV cache as in the one-after-another order, so the results are the same bits.
 * Applies to panel-weight models with hidden 2048 and the chunk attention kernel's shapes;
 * others run one chunk after another. depth 1 turns it off; depth < 1 only queries. Default
 * and maximum 8. Returns the previous depth, or -1 without a context. */
HYMT2_HIP_API int hymt2_hip_prefill_pipeline(void *impl, int depth);

/* LM head on device pointers (enqueued on the context stream): logits[r] = row r of an
 * uploaded F16/F32 weight . rmsnorm(h; norm_w, eps), each row summed sequentially in the
 * reference's order (src/model.c:887-900, src/kernels.c:1279-1300). With key != NULL also
 * folds the first-index greedy argmax over rows < n_arg into *key with atomicMax (the caller
 * zeroes *key first; token = 0xffffffff - (key & 0xffffffff)). */
HYMT2_HIP_API int hymt2_hip_head(void *impl, hy_dweight *w, const float *h_dev, const float *norm_dev, float eps,
                                 float *logits_dev, int n_arg, unsigned long long *key_dev);

/* The decode step's feed-forward input kernel on device pointers (enqueued on the context
 * stream), for one token: out[r] = SwiGLU(gate_r, up_r) with gate/up = rows of wg/wu . Q8_K(
 * rmsnorm(h; norm_w, eps)), i.e. src/model.c:870-876 for nt = 1 (RMSNorm :719-739, quantize_q8k
 * src/kernels.c:128-165, matmul_rows :1241, SiLU-gate :875). wg and wu must be uploaded
 * quantized weights of one kind and shape. */
HYMT2_HIP_API int hymt2_hip_ffn_in(void *impl, hy_dweight *wg, hy_dweight *wu, const float *h_dev,
                                   const float *norm_dev, float eps, float *out_dev);

#ifdef __cplusplus
}
#endif
#endif
