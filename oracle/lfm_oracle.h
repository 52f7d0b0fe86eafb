/*
 * lfm_oracle.h -- CPU restatement of the reference's LFM2 Q6_K CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker (or the timed CPU baseline), never as a product path.
 *
 * Every function cites the reference file:line it restates.  Paths are
 * relative to the reference repository root (Amidwestnoob/lfm2-w9100-rust).
 * Arithmetic rules (follow engine/src/lfm.rs exactly): f32 sequential sums in
 * mul_mat_weight / mul_mat_expert / rms_norm / conv / SwiGLU, f64 sums in
 * q6k_matvec and attention, built with -O2 -ffp-contract=off, no fast-math,
 * glibc expf/exp/sinf/cosf/sqrtf/powf, f32 powi as square-and-multiply.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   fp16 <-> f32        : IEEE 754, checked exhaustively against numpy float16
 *                          plus the q6k.rs:199-203 known answers.
 *   Q6_K dequant        : q6k.rs:205-250 known answers, the dequant_mirror.rs
 *                          identity over its 512 xorshift blocks, an exhaustive
 *                          per-element closed form, and the signed-zero rule.
 *   q6k_matvec (f64)    : brute force with numpy float64 and q6k.rs:252-290.
 *   argmax              : main.rs:287-317 cases restated.
 *   router / top-k      : stable-sort tie rule, numpy restatement, resident_check
 *                          properties (ids ordered by score, weights sum to 1).
 *   rms_norm, rope, attention, conv, SwiGLU, combine, full forward: closed-form
 *                          numpy restatements at small sizes and invariants
 *                          (rope preserves pair norms, softmax weights sum to 1,
 *                          conv state shift, causal prefix consistency between
 *                          one n-token forward and n one-token forwards).
 */
#ifndef LFM_ORACLE_H
#define LFM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_MAX_LAYERS 64
#define ORACLE_GGML_F32 0u
#define ORACLE_GGML_Q6_K 14u

/* Mirrors Hyperparams (engine/src/lfm.rs:31-49). */
typedef struct oracle_hparams {
    uint32_t dim, heads, head_dim, n_layers;
    uint32_t kv_heads[ORACLE_MAX_LAYERS]; /* 0 = shortconv layer, >0 = attention */
    uint32_t vocab;
    float eps, rope_theta;
    uint32_t eos;
    uint32_t n_expert, n_used, expert_ff, n_ff, dense_lead, conv_l_cache;
} oracle_hparams;

/* ---- fp16 (half 2.7.1 semantics: IEEE binary16, RNE) ---- */
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
float oracle_f16_round(float x);
void oracle_f32_to_f16_array(const float *in, uint16_t *out, size_t n);

/* ---- Q6_K (engine/src/q6k.rs) ---- */
void oracle_q6k_dequant_block(const uint8_t *blk, float *out256);
float oracle_q6k_mirror_elem(const uint8_t *blk, uint32_t k);
void oracle_q6k_dequant_row(const uint8_t *blocks, size_t n, float *out);
void oracle_q6k_matvec(const uint8_t *w, size_t in_dim, size_t out_dim,
                       const float *x, float *y);
void oracle_q6k_repack_aligned(const uint8_t *raw, size_t raw_len, uint8_t *out);

/* ---- argmax (engine/src/main.rs:112-141) ---- */
uint32_t oracle_argmax(const float *v, size_t n);
uint32_t oracle_argmax_scalar(const float *v, size_t n);

/* ---- MoE route (engine/src/lfm.rs:613-637) ---- */
void oracle_route(const float *router_logits, const float *bias, uint32_t n_expert,
                  uint32_t n_used, uint32_t *sel, float *wsel, float *scores_out);

/* ---- f32 power by square-and-multiply (f32::powi) ---- */
float oracle_powi(float a, int b);

/* ---- threads used by row-parallel loops (results are thread-count independent) ---- */
void oracle_set_threads(int n);
int oracle_get_threads(void);

/* ---- engine (engine/src/lfm.rs:67-745) ---- */
typedef struct oracle_engine oracle_engine;

oracle_engine *oracle_engine_create(const oracle_hparams *hp, uint32_t ctx, int kv_f16);
void oracle_engine_destroy(oracle_engine *e);
/* Copies the tensor bytes (GGUF layout: ne[0] fastest). */
int oracle_engine_set_tensor(oracle_engine *e, const char *name, uint32_t ggml_type,
                             const uint64_t *ne, uint32_t n_dims, const void *data,
                             size_t nbytes);
/* Pre-dequantizes every non-3D tensor to f32 (lfm.rs:165-179). */
int oracle_engine_finalize(oracle_engine *e);
/* Full forward (lfm.rs:290-694): logits of the last token into logits[vocab]. */
int oracle_forward(oracle_engine *e, const uint32_t *ids, uint32_t n, int64_t start_pos,
                   float *logits);
/* One layer's halves on a caller-held residual x[dim*n] (same code as forward). */
int oracle_run_mixer(oracle_engine *e, uint32_t layer, float *x, uint32_t n, int64_t start_pos);
int oracle_run_ffn(oracle_engine *e, uint32_t layer, float *x, uint32_t n);
/* Final norm + tied head on one residual vector (lfm.rs:676-693). */
int oracle_head(oracle_engine *e, const float *x_last, float *logits);
/* Dequantized token embedding row (lfm.rs:310-320). */
int oracle_embed(oracle_engine *e, uint32_t token, float *out_dim);

/* Recurrent state in the reference snapshot order (resident_graph.rs:572-602):
 * per layer, attention -> K then V, each head_dim*kv*valid f32 laid out
 * [t][kh][d]; shortconv -> dim*2 f32 laid out [ch][slot]. */
size_t oracle_state_bytes(const oracle_engine *e, uint32_t valid_tokens);
int oracle_snapshot(const oracle_engine *e, uint32_t valid_tokens, uint8_t *buf, size_t cap);
int oracle_restore(oracle_engine *e, uint32_t valid_tokens, const uint8_t *buf, size_t len);
void oracle_reset(oracle_engine *e);

/* The routing of one residual vector x[dim] at MoE layer l, by the same code
 * as oracle_run_ffn (lfm.rs:599-637): ids/w[n_used], scores[n_expert]
 * (sigmoid + bias), logits[n_expert] (may be NULL).  x is not changed. */
int oracle_route_layer(oracle_engine *e, uint32_t l, const float *x, uint32_t *ids, float *w,
                       float *scores, float *logits);

/* Last MoE routing decision of a layer (ids + weights), for id parity checks. */
int oracle_last_route(const oracle_engine *e, uint32_t layer, uint32_t *ids, float *w,
                      float *scores);

#ifdef __cplusplus
}
#endif
#endif
