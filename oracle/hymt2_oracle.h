/* hymt2 oracle: TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C CPU restatement of the arithmetic that the reference library
 * (zhangbo8418/hymt2) runs on its scalar ISA path (HYMT2_ISA=scalar, HYMT2_REPACK=1) for the
 * Hy-MT2 token loop. Only the test suite, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load it, and only as the checker. The product (hymt2_amd/libhymt2_hip.so) never
 * links, loads or calls anything in this directory.
 *
 * Every function names the reference file:line it follows (paths relative to the reference
 * repository root). Block layouts are byte-identical to the reference's GGUF blocks
 * (src/internal.h:21-27) and its Q8_K activation block (src/internal.h:29-41).
 *
 * Pinning: tests/test_oracle_ref.py compares every function here bit-for-bit against the
 * reference library built from its own sources (oracle/Makefile -> oracle/_ref/), and against
 * double-precision dequant references and closed-form invariants (tests/test_oracle_math.py).
 */
#ifndef HYMT2_ORACLE_H
#define HYMT2_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OC_QK 256

/* GGUF tensor type codes used by the reference (src/internal.h:46). */
enum { OC_F32 = 0, OC_F16 = 1, OC_Q8_0 = 8, OC_Q4_K = 12, OC_Q6_K = 14, OC_Q2_0C = 40, OC_STQ1_0 = 43 };

/* Q8_K activation block, 576 bytes, same byte layout as the reference's q8k_block
 * (src/internal.h:29-41): qp[256] @0 (reordered copy), d @256, sum @260, bsums[16] @264,
 * zero pad @296, qs[256] @320. */
typedef struct __attribute__((aligned(64))) {
    int8_t qp[OC_QK];
    float d;
    int32_t sum;
    int16_t bsums[OC_QK / 16];
    uint8_t pad[24];
    int8_t qs[OC_QK];
} oc_q8k;

typedef struct {
    int type;              /* OC_* */
    int k, n;              /* input dim, output rows */
    const uint8_t *data;   /* raw GGUF rows */
    const uint8_t *pk;     /* optional 2-bit panel: n * (k/256) * 64 bytes */
    const float *ps;       /* optional panel scales: n * (k/256) */
    int pshift, poff;      /* panel combine constants (STQ1_0: 0,1; Q2_0C: 1,3) */
} oc_weight;

typedef struct {
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
    oc_weight wq, wk, wv, wo, wg, wu, wd;
} oc_layer;

typedef struct {
    int n_layer, hidden, ffn, heads, kv_heads, hdim, ctx, rope_half, vocab_out;
    float eps;
    const float *rope_cos, *rope_sin; /* [ctx * rope_half] */
    oc_weight embd, outw;
    const float *out_norm;
    const oc_layer *layers;
} oc_model;

typedef struct oc_state oc_state;

/* ---- conversions ---- */
float oc_f16_to_f32(uint16_t h);
uint16_t oc_f32_to_bf16(float f);
float oc_bf16_to_f32(uint16_t h);
size_t oc_row_bytes(int type, int k);
void oc_expf_n(const float *x, float *y, int n);

/* ---- activation quantization ---- */
void oc_quantize_q8k(const float *x, int k, oc_q8k *y);

/* ---- weight formats ---- */
uint8_t oc_stq_group_codes(const uint8_t *block42, int g);
void oc_panel_repack(const oc_weight *w, uint8_t *pk, float *ps, int r0, int r1);
void oc_dequant_row(const oc_weight *w, int row, float *dst);

/* ---- matvecs: out[t * n + r] for r in [0, n), t in [0, nt) ---- */
void oc_matvec(const oc_weight *w, const float *xf, const oc_q8k *xq, int nt, float *out);
/* int32 per-block dots, enc[(t * n + r) * nb + b]; kind 0 = panel enc, 1 = Q4_K sumi,
 * 2 = Q4_K summ, 3 = Q6_K acc (the integer parts the reference combines in fp32). */
void oc_block_ints(const oc_weight *w, const oc_q8k *xq, int nt, int kind, int32_t *enc);

/* ---- attention helpers (bf16 KV) ---- */
float oc_dot_bf16(const float *q, const uint16_t *k, int n);
void oc_axpy_bf16(float *o, const uint16_t *v, float p, int n);

/* ---- model ---- */
void oc_rope_tables(int ctx, int rope_half, int hdim, float base, float alpha, float *cosv, float *sinv);
oc_state *oc_state_new(const oc_model *m);
void oc_state_free(oc_state *s);
/* Returns 0, or -1 (nothing computed) unless 1 <= nt <= 16, 0 <= pos0, pos0 + nt <= ctx and
 * every token id is a row of the embedding. */
int oc_forward(oc_state *s, const int *toks, int nt, int pos0, int want_logits, float *logits);
const float *oc_state_hidden(const oc_state *s);
int oc_argmax(const float *logits, int n);
void oc_rmsnorm(const float *x, const float *w, float *y, int dim, float eps);
/* greedy loop: prompt ids -> n_gen ids written to out; stop ids ignored. Returns n_gen. */
int oc_generate(oc_state *s, const int *prompt, int n_prompt, int n_gen, int batch, int *out);
/* gen_ids (src/model.c:914-958) from the prompt ids: prefix reuse against the ids this state's
 * cache holds, chunked prompt, greedy ids up to a stop id. Returns the ids written to out. */
int oc_gen_ids(oc_state *s, const int *prompt, int n, int max_tokens, int batch, const int *stop, int n_stop,
               int *out, int *keep_out);
void oc_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
