/*
 * lfm_hip.h -- C ABI of the MI355X (gfx950) LFM2.5-8B-A1B Q6_K token loop.
 *
 * This is the drop-in boundary that replaces the reference's Vulkan engine
 * (Amidwestnoob/lfm2-w9100-rust: engine/src/gpu_lfm.rs + gpu_lfm/resident_graph.rs
 * over engine/src/ops.rs, engine/src/kernels*.rs and engine/src/vulkan*.rs).
 * Callers that keep the reference's GGUF reader, tokenizer and CLI/JSONL code
 * bind these symbols (cgo-style plain pointers and sizes; no C++ or torch types).
 *
 * Conventions
 *   - Every call returns an int status (LFM_OK == 0); on failure a message is
 *     available from lfm_last_error() (thread-local, valid until the next call
 *     on the same thread).  No call aborts the process.
 *   - An engine is single-threaded and non-reentrant, like the reference's
 *     GpuEngine (engine/src/ops.rs:17-47 uses Cell/RefCell): one engine per
 *     thread, calls serialized by the caller.  Every engine call returns after
 *     its GPU work has completed.
 *   - Host buffers stay owned by the caller; the library copies in and writes
 *     results into caller buffers of stated capacity.
 *   - Numerical contract (engine/src/gpu_lfm.rs:8-11): signed int8 Q6_K scales,
 *     KV cache rounded to binary16 (stored as binary16), NEOX RoPE,
 *     kv head = h * kv / heads, MoE top-k with a 6.103515625e-5 weight-sum clamp,
 *     greedy argmax with ties to the lowest id and NaN never winning.
 */
#ifndef LFM_HIP_H
#define LFM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define LFM_OK 0
#define LFM_EINVAL 1    /* invalid argument or failed precondition (anyhow::ensure!) */
#define LFM_ERANGE 2    /* context / token id / capacity out of range            */
#define LFM_EDEVICE 3   /* HIP runtime or device failure                          */
#define LFM_ESTATE 4    /* call not valid in the engine's current state           */
#define LFM_EINTERNAL 5 /* library bug                                            */
#define LFM_ENOTFOUND 6 /* metadata key or tensor name not present in a GGUF file  */

#define LFM_GGML_TYPE_F32 0u
#define LFM_GGML_TYPE_Q6_K 14u
#define LFM_MAX_LAYERS 64
#define LFM_MAX_CTX 4096 /* engine/src/ops.rs:488-491 */
#define LFM_MAX_TOKEN_BATCH 64 /* forward_token batch, resident_graph.rs:95-98 */

/* Model hyper-parameters; mirrors Hyperparams (engine/src/lfm.rs:31-49) and the
 * metadata keys read by load_hyperparams (engine/src/lfm.rs:102-145). */
typedef struct lfm_hparams {
    uint32_t dim;        /* lfm2moe.embedding_length (multiple of 256)          */
    uint32_t heads;      /* lfm2moe.attention.head_count                        */
    uint32_t head_dim;   /* 64                                                  */
    uint32_t n_layers;   /* lfm2moe.block_count                                 */
    uint32_t kv_heads[LFM_MAX_LAYERS]; /* lfm2moe.attention.head_count_kv[]: 0 = conv */
    uint32_t vocab;      /* lfm2moe.vocab_size                                  */
    float eps;           /* lfm2moe.attention.layer_norm_rms_epsilon            */
    float rope_theta;    /* lfm2moe.rope.freq_base                              */
    uint32_t eos;        /* tokenizer.ggml.eos_token_id                         */
    uint32_t n_expert;   /* lfm2moe.expert_count (4..64)                        */
    uint32_t n_used;     /* lfm2moe.expert_used_count (4)                       */
    uint32_t expert_ff;  /* lfm2moe.expert_feed_forward_length (multiple of 256) */
    uint32_t n_ff;       /* lfm2moe.feed_forward_length (multiple of 256)       */
    uint32_t dense_lead; /* lfm2moe.leading_dense_block_count                   */
    uint32_t conv_l_cache; /* lfm2moe.shortconv.l_cache (3)                     */
} lfm_hparams;

typedef struct lfm_engine lfm_engine;

/* ---- library ------------------------------------------------------------- */
const char *lfm_last_error(void);
const char *lfm_version(void);
/* Number of visible HIP devices (0 when none). */
int lfm_device_count(int *count);
/* Free and total device memory in bytes; replaces the sysfs mem_info_vram_*
 * reads of bin/api_stream.rs:43-47 (co-resident headroom check). */
int lfm_device_mem_info(int device, uint64_t *free_bytes, uint64_t *total_bytes);

/* ---- engine lifecycle ---------------------------------------------------- */
/* GpuEngine::load (gpu_lfm.rs:51-115) is split into create / upload / finalize
 * so that the caller's GGUF reader (model_file.rs:100-109) streams tensors in. */
int lfm_engine_create(const lfm_hparams *hp, int device, lfm_engine **out);
/* Copies one tensor (raw GGUF bytes, ne[0] fastest) to device memory.  Names
 * and shapes are the reference's (gpu_lfm.rs:71-97, lfm.rs:330-669).  Q6_K
 * tensors are re-laid out on upload; F32 tensors are copied as-is. */
int lfm_engine_upload_tensor(lfm_engine *e, const char *name, uint32_t ggml_type,
                             const uint64_t *ne, uint32_t n_dims, const void *host,
                             size_t nbytes);
/* Verifies every tensor is present, allocates the resident state, makes the
 * prefill GEMMs' 32-row tile copies of their weights and captures the decode
 * graph.  Must precede any forward call.  A failure after the tensor check
 * (a device allocation) leaves the engine unusable: later calls to finalize
 * return LFM_ESTATE, and the engine is to be destroyed. */
int lfm_engine_finalize(lfm_engine *e);
/* GpuEngine::set_ctx (gpu_lfm.rs:117): context capacity, 1..LFM_MAX_CTX.
 * Must be called before lfm_engine_finalize (default 4096). */
int lfm_engine_set_ctx(lfm_engine *e, uint32_t ctx);
void lfm_engine_destroy(lfm_engine *e);
int lfm_engine_hparams(const lfm_engine *e, lfm_hparams *out);

/* ---- forward ------------------------------------------------------------- */
/* GpuEngine::forward (gpu_lfm.rs:243): process ids[0..n) at positions
 * start_pos.., return the last token's logits (vocab floats). */
int lfm_forward_logits(lfm_engine *e, const uint32_t *ids, uint32_t n, uint32_t start_pos,
                       float *logits, size_t logits_cap);
/* GpuEngine::forward_token (resident_graph.rs:90-101): n in 1..64; greedy next
 * id computed on the GPU; *max_logit receives the winning logit. */
int lfm_forward_token(lfm_engine *e, const uint32_t *ids, uint32_t n, uint32_t start_pos,
                      uint32_t *next, float *max_logit);
/* The greedy loop of main.rs:182-189 / api_stream.rs:67-77 resident on the
 * device: feed `first_token` at `start_pos`, then each argmax back in, for up
 * to `steps` tokens; stops after emitting nothing once the argmax equals `eos`
 * (eos >= vocab never stops).  out_tokens receives the argmax ids in order,
 * *n_out their count (the eos id itself is not stored). */
int lfm_decode_run(lfm_engine *e, uint32_t first_token, uint32_t start_pos, uint32_t steps,
                   uint32_t eos, uint32_t *out_tokens, uint32_t *n_out);
/* GpuEngine::reset_session (resident_graph.rs:105-115): zero conv state. */
int lfm_reset_session(lfm_engine *e);
/* snapshot_resident_cache (resident_graph.rs:572-602): same byte format
 * (attention layers: K then V, head_dim*kv*valid f32 in [t][kh][d] order;
 * conv layers: dim*2 f32 in [ch][slot] order). */
int lfm_snapshot_bytes(const lfm_engine *e, uint32_t valid_tokens, size_t *nbytes);
int lfm_snapshot_cache(lfm_engine *e, uint32_t valid_tokens, uint8_t *buf, size_t cap,
                       size_t *written);
/* restore_session (resident_graph.rs:119-158): exact-size input required. */
int lfm_restore_session(lfm_engine *e, uint32_t valid_tokens, const uint8_t *buf, size_t len);
/* snapshot_resident_logits (resident_graph.rs:561-568): last full logits. */
int lfm_snapshot_logits(lfm_engine *e, float *out, size_t cap);
/* Multi-token forwards (n >= 2) run the batched matrix-core prefill by default
 * (stepwise = 0); stepwise = 1 runs them as one captured decode step per token
 * instead (the reference's token-by-token equivalence, used by parity tests). */
int lfm_engine_set_prefill_mode(lfm_engine *e, int stepwise);
/* No counterpart in the reference (its weights stay Q6_K on the device): device
 * bytes this engine holds in binary16 copies of its GEMM weights, which the
 * multi-token forwards of more than 128 tokens read instead of decoding Q6_K.
 * lfm_engine_finalize makes one per weight whose sub-block scales all lie within
 * [-64, 64] (binary16 holds those weights exactly; 2.4 times the weight's Q6_K
 * bytes, about 16.4 GB for LFM2.5-8B-A1B) unless the environment sets
 * LFM_PREFILL_H16=0 or the device has no memory left for it; 0 when none. */
int lfm_engine_h16_bytes(const lfm_engine *e, uint64_t *bytes);
/* gpu.dispatch_count(): kernels launched by this engine so far. */
uint64_t lfm_dispatch_count(const lfm_engine *e);
/* device_name (gpu_lfm.rs:126-128). */
int lfm_device_name(const lfm_engine *e, char *buf, size_t cap);

/* ---- layer-level entry points (parity tests) ------------------------------
 * Run one layer's mixer half (RMSNorm -> conv or attention -> residual) or
 * FFN half (RMSNorm -> dense SwiGLU or MoE -> residual) of the decode step on
 * a host residual vector x[dim] in place, at position `pos`, with the same
 * kernels the decode graph replays (lfm.rs:330-670 one token at a time).
 * lfm_engine_last_route returns the ids/weights the last MoE kernel chose. */
int lfm_engine_run_mixer(lfm_engine *e, uint32_t layer, float *x, uint32_t pos);
int lfm_engine_run_ffn(lfm_engine *e, uint32_t layer, float *x);
int lfm_engine_last_route(lfm_engine *e, uint32_t *ids, float *weights, uint32_t cap);
/* A whole layer as the decode step runs it (resident_graph.rs:237-503 for one
 * layer): mixer, then FFN with the MoE router fused into the mixer's output
 * projection where the step fuses it, so lfm_engine_last_route then returns the
 * routing of the step's own kernels.  x_mid (dim floats, may be NULL) receives
 * the residual between the two halves, i.e. the FFN input the routing saw. */
int lfm_engine_run_layer(lfm_engine *e, uint32_t layer, float *x, uint32_t pos, float *x_mid);
/* *fused = 1 when MoE layer `layer` routes through the fused router in the
 * decode step (32 experts, dim 2048), else 0. */
int lfm_engine_fused_router(const lfm_engine *e, uint32_t layer, int *fused);

/* ---- routing audit (parity tests; no counterpart in the reference) ---------
 * The routing the reference records per layer and token (lfm.rs:613-637) as
 * the GPU computed it, so tests compare expert selections and their margins
 * with the oracle decision by decision.
 * lfm_engine_route_records copies the decode step's routing records, 144
 * words per layer (n_layers * 144 words; layer l at l * 144): ids[8], then
 * weights[8] (float bits), then the router logits [16 + e] and the selection
 * scores p + bias the kernel ranked the experts by [80 + e] (float bits), for
 * e < n_expert.  Each decode step (lfm_forward_* of one token, lfm_decode_run,
 * lfm_engine_run_layer / _run_ffn) rewrites the records of the MoE layers it
 * runs; dense layers stay zero. */
int lfm_engine_route_records(lfm_engine *e, uint32_t *words, size_t cap_words);
/* on = 1 makes every later multi-token (matrix-core) forward keep its routing:
 * per MoE layer and token row, ids[4], weights[4] and the router logits
 * [n_expert] the selection was made from.  The first enable allocates the log
 * on the device (n_layers * ctx * (32 + 4 * n_expert) bytes).
 * lfm_engine_prefill_routes returns layer `layer`'s log of the last such call:
 * token rows *first .. *first + *n - 1 (the last layer routes only the last
 * row), ids[*n][4], w[*n][4] and, when *has_logits, logits[*n][n_expert]
 * (logits may be NULL).  LFM_ESTATE while the log was never enabled. */
int lfm_engine_set_route_log(lfm_engine *e, int on);
int lfm_engine_prefill_routes(lfm_engine *e, uint32_t layer, uint32_t *first, uint32_t *n,
                              int *has_logits, uint32_t *ids, float *w, float *logits,
                              size_t cap_rows);

/* Mean duration of the routed MoE gate/up kernel (the largest share of a decode
 * step), timed with HIP events over one graph of `reps` rounds across every MoE
 * layer's routed experts; *bytes_per_launch = its algorithmic HBM bytes. */
int lfm_engine_time_moe_gateup(lfm_engine *e, uint32_t reps, float *us_per_launch,
                               uint64_t *bytes_per_launch);

/* Mean duration of the final-norm + tied-head kernel (vocab x dim Q6_K, the
 * largest single matvec of a step), timed with HIP events over one graph of
 * `reps` rounds rotating `ncopies` (1..8) copies of the embedding planes (the
 * library allocates the extra copies and frees them before returning);
 * *bytes_per_launch = its algorithmic HBM bytes.  No reference counterpart:
 * measurement only. */
int lfm_engine_time_head(lfm_engine *e, uint32_t ncopies, uint32_t reps, float *us_per_launch,
                         uint64_t *bytes_per_launch);

/* ---- device buffers (op-level tests and measurement) --------------------- */
int lfm_dev_alloc(size_t nbytes, void **ptr);
int lfm_dev_free(void *ptr);
int lfm_memcpy_htod(void *dst, const void *src, size_t nbytes);
int lfm_memcpy_dtoh(void *dst, const void *src, size_t nbytes);
int lfm_dev_synchronize(void);

/* ---- Q6_K operator API (GpuOps::q6k_matmul, engine/src/ops.rs:340-374) ----
 * Q6_K device layout: a tensor of `rows` rows of in_dim/256 superblocks is
 * stored as four planes (ql 128 B, qh 64 B, scales 16 B, d 2 B per block, 210
 * B per block in total, the same size as GGUF).  lfm_q6k_pack converts raw
 * GGUF bytes (host) into that layout (host). */
size_t lfm_q6k_nbytes(uint64_t rows, uint64_t in_dim);
int lfm_q6k_pack(const void *raw, uint64_t rows, uint64_t in_dim, void *packed);
int lfm_q6k_unpack(const void *packed, uint64_t rows, uint64_t in_dim, void *raw);
/* Bit-exact dequantization of a packed device tensor to f32 (device). */
int lfm_q6k_dequant(const void *packed_dev, uint64_t rows, uint64_t in_dim, float *out_dev,
                    void *stream);
/* y[r] = sum_k W[r,k] * x[k] on device buffers (q6k_matvec, q6k.rs:167-183). */
int lfm_q6k_matvec(const void *packed_dev, uint64_t rows, uint64_t in_dim, const float *x_dev,
                   float *y_dev, void *stream);
/* Launch the matvec `iters` times, rotating over `ncopies` packed weight
 * copies laid out back to back from packed_dev, and return the mean ms per
 * launch measured with HIP events on the launch stream (rotation defeats the
 * 256 MB Infinity Cache when ncopies * size exceeds it). */
int lfm_q6k_matvec_time(const void *packed_dev, uint32_t ncopies, uint64_t rows, uint64_t in_dim,
                        const float *x_dev, float *y_dev, uint32_t iters, float *ms_per_launch);

/* Measurement utility with no counterpart in the reference: mean time of a
 * plain device copy of `bytes` (multiple of 16) over `reps` launches -- the
 * achievable HBM rate that roofline figures are read against, and the known
 * traffic that scales the memory counters of a profile. */
int lfm_copy_time(uint64_t bytes, uint32_t reps, float *us_per_copy);

/* Prefill GEMM on the matrix cores: y[t][r] = sum_k W[r][k] * x[t][k] for T
 * activation rows x (f32 [T][in_dim], device) into y (f32 [T][rows], device);
 * the multi-token q6k_prompt path of engine/src/ops.rs:350-373.  in_dim is a
 * multiple of 256 up to 8192 and (T + 31) * in_dim * 2 bytes stays below 2 GiB
 * (the kernels address the binary16 activation copies with 32-bit offsets);
 * LFM_EINVAL otherwise.  This op-level entry point builds its scratch on every
 * call: it allocates the binary16 activation copies, the split-K partial sums
 * (T <= 128) and a 32-row tile copy of the weight (ceil(rows / 32) * in_dim /
 * 256 * 6720 bytes), runs the tile pack kernel, waits for `stream` and frees
 * them, so a caller that loops over it pays for the allocations and the repack
 * each time.  The engine's prefill keeps its
 * tile copies from lfm_engine_finalize and never repacks. */
int lfm_q6k_gemm(const void *packed_dev, uint64_t rows, uint64_t in_dim, const float *x_dev,
                 uint32_t T, float *y_dev, void *stream);

/* ---- argmax (engine/src/kernels/persistent.rs:11-53 semantics) ------------ */
int lfm_argmax(const float *v_dev, uint32_t n, uint32_t *index, float *value);
/* No counterpart in the reference.  The argmax of lfm_argmax (same kernels, same
 * result) for callers that cannot allocate device memory: tight serving loops and
 * harnesses that forbid hipMalloc.  It allocates nothing: its state block and
 * first-stage partials live in a fixed 8448-byte device array of the library's
 * own code object, one copy per device, whose address the device's first
 * launching call (lfm_engine_create, lfm_argmax, ...) takes; before that it
 * returns LFM_ESTATE.  The array size does not depend on n (at most 1024
 * first-stage workgroups, grid-stride beyond).  Every call on a device shares
 * that device's array: calls that overlap on one device race. */
int lfm_argmax_noalloc(const float *v_dev, uint32_t n, uint32_t *index, float *value);

/* ---- synthetic model (seeded; identical bytes on every host) -------------- */
typedef struct lfm_tensor_desc {
    char name[96];
    uint32_t ggml_type;
    uint32_t n_dims;
    uint64_t ne[4];
    uint32_t kind;   /* 0 = Q6_K weight, 1 = norm 1+N(0,s), 2 = N(0,s), 3 = zeros */
    float sigma;
} lfm_tensor_desc;
typedef struct lfm_synth_opts {
    uint64_t seed;
    float d_sigma;      /* Q6_K super-block scale d ~ N(0, d_sigma) as binary16  */
    float norm_sigma;   /* norm weights ~ 1 + N(0, norm_sigma)                    */
    float router_sigma; /* ffn_gate_inp ~ N(0, router_sigma)                      */
    float bias_sigma;   /* exp_probs_b ~ N(0, bias_sigma); 0 => zeros            */
    float conv_sigma;   /* shortconv.conv ~ N(0, conv_sigma)                      */
    uint32_t full_scales; /* 0: Q6_K sub-block scales uniform in [-32, 31]; 1: over the
                           * whole int8 range, one per super-block at -128 (the form
                           * real model files have: ggml's quantizer maps each block's
                           * largest-magnitude scale to -128)                      */
} lfm_synth_opts;
void lfm_synth_default_opts(lfm_synth_opts *o);
int lfm_model_tensor_count(const lfm_hparams *hp);
int lfm_model_tensor_desc(const lfm_hparams *hp, const lfm_synth_opts *o, int index,
                          lfm_tensor_desc *out);
size_t lfm_tensor_nbytes(const lfm_tensor_desc *d);
/* Fill `out` (lfm_tensor_nbytes bytes) with the tensor's seeded content. */
int lfm_synth_tensor(const lfm_synth_opts *o, const lfm_tensor_desc *d, void *out, size_t cap,
                     int threads);
/* Uniform random Q6_K blocks / normal f32 values (seeded streams). */
int lfm_synth_q6k_blocks(uint64_t seed, const char *stream, uint64_t nblocks, float d_sigma,
                         uint8_t *out, int threads);
/* The same with the full_scales choice of lfm_synth_opts. */
int lfm_synth_q6k_blocks_ex(uint64_t seed, const char *stream, uint64_t nblocks, float d_sigma,
                            int full_scales, uint8_t *out, int threads);
int lfm_synth_normal_f32(uint64_t seed, const char *stream, uint64_t n, float mean,
                         float sigma, float *out, int threads);
/* Generate every tensor of the model and upload it (convenience for benches). */
int lfm_engine_load_synthetic(lfm_engine *e, const lfm_synth_opts *o, int threads);

/* ---- GGUF v3 model files --------------------------------------------------
 * Reader: parser/src/gguf.rs:299-440 (parse: header, metadata, tensor infos and
 * every check it makes) and engine/src/model_file.rs:30-186 (ModelFile: tensor
 * table with absolute offsets, positioned tensor reads, typed metadata access).
 * A handle is read-only after open and may be shared between threads. */
#define LFM_GGUF_TYPE_U8 0u
#define LFM_GGUF_TYPE_I8 1u
#define LFM_GGUF_TYPE_U16 2u
#define LFM_GGUF_TYPE_I16 3u
#define LFM_GGUF_TYPE_U32 4u
#define LFM_GGUF_TYPE_I32 5u
#define LFM_GGUF_TYPE_F32 6u
#define LFM_GGUF_TYPE_BOOL 7u
#define LFM_GGUF_TYPE_STRING 8u
#define LFM_GGUF_TYPE_ARRAY 9u
#define LFM_GGUF_TYPE_U64 10u
#define LFM_GGUF_TYPE_I64 11u
#define LFM_GGUF_TYPE_F64 12u
#define LFM_GGUF_MAX_DIMS 8

typedef struct lfm_gguf lfm_gguf;
/* parser::gguf::TensorInfo (gguf.rs:58-70) + model_file::TensorInfo (model_file.rs:7-14). */
typedef struct lfm_gguf_tensor {
    const char *name;     /* valid until lfm_gguf_close                          */
    uint32_t ggml_type;   /* 0 = F32, 14 = Q6_K, ...                             */
    uint32_t n_dims;
    uint64_t ne[LFM_GGUF_MAX_DIMS]; /* GGUF order: ne[0] is the row length       */
    uint64_t offset;      /* as stored: relative to the data section             */
    uint64_t file_offset; /* absolute: data_offset + offset                      */
    uint64_t nbytes;
} lfm_gguf_tensor;
/* One metadata value (parser::gguf::Value, gguf.rs:40-55). */
typedef struct lfm_gguf_value {
    uint32_t type;      /* LFM_GGUF_TYPE_*                                        */
    uint32_t elem_type; /* ARRAY: type of every element                           */
    uint64_t u64;       /* U8, U16, U32, U64, BOOL                                */
    int64_t i64;        /* I8, I16, I32, I64                                      */
    double f64;         /* F32, F64                                               */
    const char *str;    /* STRING: UTF-8 bytes, NUL-terminated, valid until close */
    uint64_t len;       /* STRING: byte length; ARRAY: element count              */
} lfm_gguf_value;

int lfm_gguf_open(const char *path, lfm_gguf **out);               /* ModelFile::open     */
int lfm_gguf_parse_memory(const void *data, size_t len, lfm_gguf **out); /* gguf::parse  */
void lfm_gguf_close(lfm_gguf *g);
int lfm_gguf_header(const lfm_gguf *g, uint32_t *version, uint32_t *alignment,
                    uint64_t *data_offset, uint64_t *n_kv, uint64_t *n_tensors);
/* Keys in byte-wise order (the reference's BTreeMap); index < n_kv. */
int lfm_gguf_meta_key(const lfm_gguf *g, uint64_t index, const char **key);
int lfm_gguf_meta_get(const lfm_gguf *g, const char *key, lfm_gguf_value *out);
int lfm_gguf_meta_array_get(const lfm_gguf *g, const char *key, uint64_t index,
                            lfm_gguf_value *out);
/* Typed accessors with the reference's conversions (model_file.rs:131-182). */
int lfm_gguf_meta_u32(const lfm_gguf *g, const char *key, uint32_t *out);
int lfm_gguf_meta_f32(const lfm_gguf *g, const char *key, float *out);
int lfm_gguf_meta_str(const lfm_gguf *g, const char *key, char *buf, size_t cap, size_t *len);
int lfm_gguf_meta_u32_array(const lfm_gguf *g, const char *key, uint32_t *out, size_t cap,
                            size_t *len);
int lfm_gguf_tensor_info(const lfm_gguf *g, uint64_t index, lfm_gguf_tensor *out);
int lfm_gguf_find_tensor(const lfm_gguf *g, const char *name, uint64_t *index); /* tensor() */
/* read_tensor_into (model_file.rs:100-109): len must equal the tensor's nbytes. */
int lfm_gguf_read_tensor(const lfm_gguf *g, const char *name, void *dst, size_t len);
int lfm_gguf_read_tensor_range(const lfm_gguf *g, const char *name, uint64_t byte_off,
                               void *dst, uint64_t len); /* model_file.rs:111-122 */
/* load_hyperparams (engine/src/lfm.rs:102-145).  strict != 0 also requires the
 * reference's fixed geometry (dim 2048, 32 heads, 24 layers, vocab 128000,
 * 32 experts, top-4, expert_ff 1792), as the reference always does. */
int lfm_gguf_hparams(const lfm_gguf *g, int strict, lfm_hparams *out);
/* GpuEngine::load's staging loop (gpu_lfm.rs:64-97): uploads every F32 and Q6_K
 * tensor of the file; call before lfm_engine_finalize. */
int lfm_engine_load_gguf(lfm_engine *e, const lfm_gguf *g);
/* ModelFile::open + GpuEngine::load + set_ctx (gpu_lfm.rs:51-120): a finalized
 * engine; ctx 0 keeps the default 4096. */
int lfm_engine_open_gguf(const char *path, int device, uint32_t ctx, int strict,
                         lfm_engine **out);

/* Writer (no counterpart in the reference, whose tests build GGUF bytes by hand,
 * gguf.rs:450-553): metadata and tensor table first, then begin() writes the
 * header, then each tensor's bytes, then finish().  Key "general.alignment" (U32,
 * a power of two) sets the data alignment, default 32. */
typedef struct lfm_gguf_writer lfm_gguf_writer;
int lfm_gguf_writer_create(lfm_gguf_writer **out);
void lfm_gguf_writer_free(lfm_gguf_writer *w);
/* Scalar types only; value points to the little-endian value (BOOL: one byte 0/1). */
int lfm_gguf_writer_set_scalar(lfm_gguf_writer *w, const char *key, uint32_t type,
                               const void *value);
int lfm_gguf_writer_set_string(lfm_gguf_writer *w, const char *key, const char *s, uint64_t len);
int lfm_gguf_writer_set_array(lfm_gguf_writer *w, const char *key, uint32_t elem_type,
                              const void *values, uint64_t count);
/* lens may be NULL for NUL-terminated strings. */
int lfm_gguf_writer_set_string_array(lfm_gguf_writer *w, const char *key,
                                     const char *const *strs, const uint64_t *lens,
                                     uint64_t count);
/* The lfm2moe.* keys load_hyperparams reads, plus general.architecture. */
int lfm_gguf_writer_set_hparams(lfm_gguf_writer *w, const lfm_hparams *hp);
int lfm_gguf_writer_add_tensor(lfm_gguf_writer *w, const char *name, uint32_t ggml_type,
                               uint32_t n_dims, const uint64_t *ne, uint64_t *index);
int lfm_gguf_writer_begin(lfm_gguf_writer *w, const char *path);
int lfm_gguf_writer_write_tensor(lfm_gguf_writer *w, uint64_t index, const void *data,
                                 uint64_t nbytes);
int lfm_gguf_writer_finish(lfm_gguf_writer *w);
/* The seeded synthetic model as a GGUF file (o NULL = default options). */
int lfm_gguf_write_synthetic(const char *path, const lfm_hparams *hp, const lfm_synth_opts *o,
                             int threads);

/* ---- binary16 helpers (IEEE RNE) ------------------------------------------ */
uint16_t lfm_f32_to_f16(float f);
float lfm_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif
