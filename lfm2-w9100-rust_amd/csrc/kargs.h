// kargs.h -- kernel argument blocks shared by the host launcher (engine.cpp)
// and the gfx950 kernels (lfm_kernels.hip).  Every kernel takes exactly one of
// these structs by value, so hipModuleLaunchKernel passes {&args}.
#pragma once
#include <stdint.h>

// A Q6_K tensor in the device plane layout: `rows` rows of `nb` super-blocks.
// Planes, back to back from `base`:
//   ql  rows*nb*128 B  per block: 8 lane chunks of 16 B; chunk c holds
//                      ql[h*64+l0 .. +8] ++ ql[h*64+32+l0 .. +8] (h=c/4, l0=(c%4)*8)
//   qh  rows*nb*64  B  GGUF order
//   sc  rows*nb*16  B  per block: 4 groups of 4 scales; group p holds
//                      sc[(p/2)*8 + (p%2) + 2*s] for s = 0..3
//   d   rows*nb*2   B  binary16 super-block scales
struct Q6T {
    const uint8_t *base;
    uint32_t rows;
    uint32_t nb;
};

// Device-resident decode state.  Kernels read the token and position from
// here, so one captured graph serves every position.
struct DevState {
    uint32_t tok;       // token fed to the current step
    uint32_t pos;       // its absolute position
    uint32_t halt;      // nonzero: every kernel of a step returns at once
    uint32_t step;      // next slot of out_tokens
    uint32_t eos;       // argmax == eos sets halt (>= vocab: never)
    uint32_t cursor;    // prompt cursor used by k_advance
    uint32_t n_ids;     // prompt length in ids
    uint32_t last_token;
    float last_value;
    uint32_t fault;     // nonzero: a fused kernel's bounded handoff wait timed out
    uint32_t pad[5];
    uint32_t gen;       // step generation: the last kernel of every step adds 1;
                        // the host never rewrites it (fused kernels' handoff tags)
};                      // 64 bytes
static_assert(sizeof(DevState) == 64, "DevState is 64 bytes");

// Where a kernel's input vector comes from.
struct XSrc {
    const float *x;      // residual / activation vector (ignored when embed)
    const float *norm_w; // RMSNorm weight, nullptr = no norm
    float eps;
    uint32_t embed;      // 1: x = dequantized row DevState::tok of `emb`
    Q6T emb;
    float *x_out;        // embed: workgroup 0 writes x here (the residual)
};

// Rows per workgroup of the long-row matvec (k_q6_matvec_long).
#define LONG_ROWS 8

struct MatvecArgs {      // y = W x  (mode 0)  or  y += W x  (mode 1)
    Q6T w;
    XSrc src;
    float *y;
    uint32_t in_dim;
    uint32_t mode;
    DevState *st;        // nullable
};

struct ConvInprojArgs {  // LFM2 gated short conv, decode: in_proj + conv + gate
    Q6T w;               // in_proj, rows 3*dim (B, C, x)
    XSrc src;
    const float *conv_w; // [dim][3]
    float *state;        // [dim][2]
    float *y;            // gated output [dim]
    uint32_t dim;
    DevState *st;
};

struct QkvArgs {
    Q6T wq, wk, wv;
    XSrc src;
    float *qkv;          // [dim + 2*hdkv]
    uint32_t dim, hdkv;
    DevState *st;
};

struct AttnArgs {
    const float *qkv;
    const float *q_norm, *k_norm;
    const float *rope;         // [ctx][32] (cos, sin) of theta = pos * tscale^p
    float eps, scale;
    uint16_t *kcache, *vcache; // [kv][ctx][64] binary16
    float *part;               // [kv][nchunk][4][66]: max, sum, o[64]
    uint32_t ctx, heads, kv, nchunk;
    DevState *st;
};

struct AttnMergeArgs {
    const float *part;
    float *out;                // [heads*64]
    uint32_t heads, kv, nchunk;
    DevState *st;
};

// Router logits of the MoE layer; the top-k itself is taken by every consumer
// wave from these logits (identical result everywhere, no cross-workgroup sync).
struct RouterArgs {
    XSrc src;
    const float *w;      // [n_expert][dim] f32
    float *logits;       // [n_expert]
    uint32_t dim, n_expert;
    DevState *st;
};

struct Route {
    const float *logits; // nullptr = dense layer (or the fused router below)
    const float *bias;
    uint32_t n_expert, n_used;
    uint32_t *sel_out;   // routing record of the layer (ROUTE_REC_WORDS, see below), one wave writes it
    const float *rpart;  // fused router: expert partial sums, [ROUTE_QUADS][ROUTE_PARTS] float4
    const float *rss;    // fused router: partial sums of x_new^2 [ROUTE_PARTS]
    const float *xw;     // fused router: x_new * w_norm, the FFN's input before 1/rms [width]
};

// Routing record of one MoE layer in the decode step, written by the gate/up
// kernel and read by the down projection: ids[8], weights[8] (float bits, the
// normalized picks), then per expert e < n_expert the router logit at
// [ROUTE_REC_LOGITS + e] and the selection score p + bias it was ranked by at
// [ROUTE_REC_SCORES + e] (float bits).  The step keeps one record per layer.
#define ROUTE_REC_LOGITS 16
#define ROUTE_REC_SCORES 80
#define ROUTE_REC_WORDS 144

// Fused router (the model's 32 experts at width 2048): the output projection
// before the FFN runs ROUTE_PARTS workgroups of ROUTE_ROWS rows; each leaves
// the partial dots sum_r R[e][r] * (x_new[r] * w_norm[r]) and sum_r x_new[r]^2
// of its rows, which the gate/up kernel adds up.  The expert partials are
// stored quad-major: float4 q of workgroup p (experts 4q .. 4q+3) at
// rpart[q * ROUTE_PARTS + p], so a workgroup writes 8 aligned 16-byte pieces and
// a reader wave sums one quad's column with one float4 per lane and row.
#define ROUTE_EXPERTS 32
#define ROUTE_QUADS (ROUTE_EXPERTS / 4)
#ifndef ROUTE_ROWS
#define ROUTE_ROWS 8
#endif
#define ROUTE_WIDTH 2048
#define ROUTE_PARTS (ROUTE_WIDTH / ROUTE_ROWS)

struct MatvecRouteArgs { // y += W x (mode 1) and the router partial sums of the new y
    MatvecArgs m;
    const float *rwt;    // router weights transposed, [rows][ROUTE_EXPERTS] f32
    const float *rnorm;  // RMSNorm weight of the FFN input [rows]
    float *rpart;        // [ROUTE_QUADS][ROUTE_PARTS] float4 (see above)
    float *rss;          // [ROUTE_PARTS]
    float *xw;           // [rows]: y_new * rnorm, read by the gate/up kernel
};

struct GateUpArgs {      // sw = silu(Wg h) * (Wu h), dense or routed
    Q6T wg, wu;
    XSrc src;
    Route route;
    float *sw;           // [n_used][ff] or [ff]
    uint32_t ff;
    DevState *st;
};

struct MoeDownArgs {     // x[k] += sum_r w_r * (Wd[e_r] sw_r)[k]
    Q6T wd;              // rows n_expert*dim
    const float *sw;     // [n_used][ff]
    Route route;
    float *x;
    uint32_t dim, ff;
    DevState *st;
};

struct HeadArgs {        // logits = E rmsnorm(x), per-workgroup greedy argmax partials
    Q6T emb;
    XSrc src;
    float *logits;       // [vocab]
    float *partial;      // [grid][2]
    uint32_t vocab;
    DevState *st;
};

struct ArgmaxArgs {      // per-workgroup argmax partials of a plain vector
    const float *v;
    float *partial;
    uint32_t n;
    DevState *st;
};

// A forward call's result, stored by k_argmax_final straight into pinned host
// memory (read once the stream has synchronized: no copy back).  token is
// ~0u until the kernel has written it.
struct HostResult {
    uint32_t token;
    float value;
    uint32_t fault; // DevState::fault when the result was stored
    uint32_t pad;
};

struct FinalArgs {       // reduce partials; decode step: store, feed back, advance
    const float *partial;
    uint32_t n_partial;
    uint32_t *out_tokens;
    uint32_t advance;
    DevState *st;
    HostResult *host;    // nullable: also store the result here (device address of pinned memory)
};

struct AdvanceArgs {
    const uint32_t *ids;
    DevState *st;
};

struct DequantArgs {
    Q6T w;
    float *out;
    uint32_t in_dim;
};

struct CopyArgs { // plain device copy (achievable-bandwidth reference)
    const uint4 *src;
    uint4 *dst;
    uint64_t n16; // 16-byte units
};

// ---- prefill (multi-token) path ----------------------------------------------
// RMSNorm (optional) + binary16 hi/lo split of T rows of K floats, with a per-row
// power-of-two scale so that |x / scale| < 2^14 (hi/lo then hold ~22 bits).
// Activations for the small-call GEMMs (calls of up to GEMM_TOKENS tokens) are
// token-blocked: element k of logical row L at
//   ((L / 32) * (K / 8) + k / 8) * 256 + (L % 32) * 8 + k % 8   (binary16),
// so the B fragment of 32 rows and 8 k's is 512 contiguous bytes.
__host__ __device__ inline size_t blocked_index(uint32_t L, uint32_t k, uint32_t K)
{
    return (((size_t)(L >> 5) * (K >> 3) + (k >> 3)) << 8) + ((L & 31) << 3) + (k & 7);
}

#define SPLIT_ROWMAJOR 0 // hi / lo [T][K] (large calls)
#define SPLIT_BLOCKED 1  // blocked, logical row = source row
#define SPLIT_GROUPED 2  // blocked, logical rows of the expert slots (see SplitArgs)

struct SplitArgs {
    const float *x;      // [T][K]
    const float *norm_w; // nullable
    float eps;
    uint16_t *hi, *lo;   // binary16, layout by `mode`
    float *scale;        // [T], per source row
    // blocked modes: the scale of logical row L's half-block h (k = 128 h .. + 127)
    // at bscale[L * (K / 128) + h], which the small-call GEMMs read (a split row has
    // one scale: it is written to each of the row's half-blocks)
    float *bscale;
    uint32_t T, K;
    uint32_t mode;       // SPLIT_*
    // SPLIT_GROUPED: source row t feeds slots s = t * spr .. t * spr + spr - 1 (spr 4:
    // token rows of the gate/up input, spr 1: slot rows of the down input); slot s
    // with rank s % 4 < n_used goes to logical row sel[s] * rpe + pos[s] (expert
    // sel[s], index pos[s] in its token list, rpe rows reserved per expert)
    const uint32_t *sel;
    uint32_t *pos;
    uint32_t spr, n_used, rpe;
    // SPLIT_GROUPED with tok set (spr 4, T <= 256 rows, n_expert <= 64): pos is
    // formed here from sel instead of read, together with k_route_group's lists
    // (tok[e][i] = token, slot[e][i] = token * 4 + rank in token order, counts[e]),
    // so that no separate grouping launch precedes the split
    uint32_t *tok, *slot, *counts;
    uint32_t list_stride, n_expert;
    // nullable (with tok): workgroup t routes token t itself from the preceding
    // reduce's router partials (rpart / rss, nparts per token; k_route_topk's rule:
    // logit = dot / sqrt(sum x^2 / K + eps), rbias added for the choice), writes
    // sel_out / wsel_out, and takes each chosen expert's list index from counts[e]
    // (zeroed by that reduce) with an atomic add: the lists are then in arrival
    // order, which changes where a token's row sits in its expert's tile but not
    // what is computed for it
    const float *rpart, *rss, *rbias;
    uint32_t *sel_out;
    float *wsel_out;
    float *logit_out;    // nullable: the router logits [T][n_expert] (routing log)
    uint32_t nparts;
    // nullable (small calls): before the split, row t of x first gets the down
    // projection's ranks combined into it as k_reduce_combine does (x += sum_r
    // cwsel[t][r] (sum_s cpart[s][t*4 + r]), rank then slice order), written back
    const float *cpart, *cwsel;
    float *cx;
    uint32_t cksplit, cn_used;
    // nullable: the workgroups also copy copy_n floats (a multiple of 4, 16-byte
    // aligned) from copy_src to copy_dst (the short conv's new state, written by the
    // kernel before this one)
    const float *copy_src;
    float *copy_dst;
    uint32_t copy_n;
};

// Q6_K weights in 32-row tiles, the prefill GEMMs' copy (the matvecs read the
// row-major planes of Q6T).  The matrix is `groups` slices of R rows (experts, or
// one); tile t covers rows 32 (t % gtiles) .. + 31 of slice t / gtiles, gtiles =
// ceil(R / 32), rows past R zero.  Tile-block tb = t * nb + kb holds those rows'
// Q6_K block kb, as four planes over all tiles * nb tile-blocks, each ordered so
// that lane l = 32 p + r of a wave (row r) loads one contiguous stretch.  In terms
// of row r's block in the Q6T planes:
//   ql [tb][q < 4][l][16 B]  code words X0 .. X3 of its chunk 2q + p (l0 = 8 (c % 4)
//                            in half c / 4 of the block)
//   qh [tb][q < 4][l][8 B]   code words X4, X5 of that chunk
//   The chunk's 32 codes are the 4 sub-blocks' codes of l = l0 .. l0 + 7; word
//   X(2s + w), s < 3, byte b holds l = l0 + 4w + b's sub-block s code in bits 2..7
//   and bits 2s, 2s + 1 of its sub-block 3 code in bits 0..1 (6 bits per code, as
//   in the Q6_K planes: k_q6_tile_pack's code_words).
//   sc [tb][h < 2][r][8 B]   its scale groups 2h, 2h + 1, each int8 scale stored as
//                            sc + 128 (128, a zero scale, throughout a block whose d is
//                            zero: such a block contributes zero weights)
//   d  [tb][r][2 B]          its d
// 6720 B per tile-block, 210 B per row and block as in the row-major planes.
#define TILE_QL 4096u
#define TILE_QH 2048u
#define TILE_SC 512u
#define TILE_D 64u
#define TILE_BYTES (TILE_QL + TILE_QH + TILE_SC + TILE_D)
struct Q6Tiles {
    const uint8_t *base;
    uint32_t tiles;  // over all slices
    uint32_t nb;     // Q6_K blocks per row
    uint32_t gtiles; // tiles per slice
    uint32_t rows;   // rows per slice (R)
    uint32_t wide;   // some sub-block scale (of a block with d != 0) lies outside
                     // [-64, 64]: its weights sc (q - 32) can exceed 2048 in
                     // magnitude and need the GEMMs' split-scale (_x) kernels
    const uint8_t *h16; // nullable: the binary16 fragment copy below (not wide only)
};

// The binary16 fragment copy of a Q6Tiles (the large-call GEMMs' A operands,
// decoded once): tile-block tb holds the 32 rows x 256 k integer weights
// sc (q - 32) of its rows' block, exact in binary16 for scales within [-64, 64],
// as 16 k-steps of 16 k: k-step j of the block is 1 KB at byte 1024 j, lane
// l = 32 p + r of a wave at 16 l holding row r's weights k = 16 j + 8 p .. + 7,
// i.e. the A fragment of v_mfma_f32_32x32x16_f16 for that k-step.  The block
// scale d stays in the Q6Tiles d plane.
#define TILE_H16 16384u

struct TilePackArgs {   // row-major planes -> Q6Tiles
    Q6T src;            // groups * group_rows rows
    uint8_t *dst;
    uint32_t group_rows, gtiles, tiles;
    uint32_t *wide;     // set to 1 when a scale outside [-64, 64] is seen (d != 0)
};

struct TileH16Args {    // Q6Tiles -> its binary16 fragment copy
    Q6Tiles src;
    uint8_t *dst;       // src.tiles * src.nb * TILE_H16 bytes
};

// C[slot(n)][col0 + r] (+)= scale[tok(n)] * sum_k W[z*zrows + r][k] * X[tok(n)][k]
// for r < zrows, n < count; blockIdx.z = z selects a weight slice (expert) and
// its token list (grouped GEMM).  Plain GEMM: zrows = the rows of w, lists null.
struct GemmArgs {
    Q6Tiles w;
    Q6Tiles w2;             // pair kernel: the up weight (gate in w), same shape
    const uint16_t *x_hi, *x_lo;
    const float *xscale;    // large calls: per activation row
    // small calls: per logical (blocked) row L and 128-wide half-block h of K, at
    // bscale[L * (K / 128) + h]: row L's activations of half-block h were stored
    // divided by it (a power of two)
    const float *bscale;
    // small-call pair form, unsplit (ksplit 1), y_hi set: the SwiGLU output is stored
    // binary16 hi + lo in the blocked layout of width zrows instead of fp32 in c: token
    // column n of group z is logical row (tok ? z * rpz : 0) + n, each 128 rows of a
    // workgroup with the power-of-two scale of their largest magnitude (y_bscale, as
    // bscale above), so that it feeds the next small-call GEMM with no split launch
    uint16_t *y_hi, *y_lo;
    float *y_bscale;
    const uint32_t *tok;    // [z][list_stride] activation rows, nullable
    const uint32_t *slot;   // [z][list_stride] output rows, nullable
    const uint32_t *counts; // [z] token counts, nullable (then ntok)
    uint32_t ntok, list_stride, zrows;
    float *c;
    uint32_t ldc, col0, mode;
    // split over K (ksplit > 1): grid z = nz groups x ksplit slices; slice s covers
    // Q6_K blocks [s nb / ksplit, (s + 1) nb / ksplit) and writes its fp32 sums to
    // part[((s * (pair ? 2 : 1) + weight) * part_rows + out_row) * zrows + row]
    float *part;
    uint32_t ksplit, nz, part_rows;
    uint32_t rpz;           // small calls, grouped: blocked activation rows per group (x 32)
};

struct GemmReduceArgs {    // c (+)= sum_s part[s] in slice order; pair: silu(g) * u
    const float *part;
    float *c;
    uint32_t ksplit, pair, part_rows, zrows, ldc, col0, mode;
    uint32_t n_used;       // grouped: out_row = token * 4 + rank, ranks >= n_used unused; 0 = all
    // Router partials (rw nullable; ungrouped, non-pair, zrows a multiple of 256):
    // workgroup (b, t), rows 256 b .. 256 b + 255 of token t, leaves the partial dots
    // sum_r rw[e][r] * (c_new[r] * rnorm[r]) of the n_expert (<= 64) experts at
    // rpart[(t * nb + b) * n_expert + e] and sum_r c_new[r]^2 at rss[t * nb + b]
    // (nb = zrows / 256), from which k_route_topk forms the next FFN's logits.
    const float *rnorm, *rw;
    float *rpart, *rss;
    uint32_t n_expert;
    uint32_t *counts; // nullable (with rw): workgroup (0, 0) zeroes counts[0 .. n_expert)
};

struct ReduceCombineArgs { // x[t] += sum_r w[t][r] * (sum_s part[s][t*4 + r]), rank then slice order
    const float *part;       // [ksplit][T*4][dim]
    const float *wsel;       // [T][4]
    float *x;                // [T][dim]
    uint32_t ksplit, T, dim, n_used;
};

struct ConvPrefillArgs {  // gated short conv over T tokens, parallel in t
    const float *bcx;     // [ksplit][T][3*dim] in_proj rows B, C, X (ksplit > 1: the
                          // split-K partial sums, added here in slice order)
    const float *conv_w;  // [dim][3]
    const float *state;   // [dim][2] before the chunk
    float *state_next;    // [dim][2] after it (copied over `state` by the next split)
    float *y;             // [T][dim]
    uint32_t T, dim, ksplit;
    // nullable (small calls): y stored binary16 hi + lo in the blocked layout (logical
    // row t, width dim) with the power-of-two scale of each 128 channels' largest
    // magnitude at y_bscale[t * (dim / 128) + ch / 128], instead of fp32 in y, so
    // that the output projection reads it with no split launch
    uint16_t *y_hi, *y_lo;
    float *y_bscale;
};

struct RopeKvArgs {       // per token: q/k head norm + RoPE, K/V to the binary16 cache
    float *qkv;           // [T][dim + 2*hdkv], the rotated q written here
    const float *src;     // [ksplit][T][dim + 2*hdkv] the projection (ksplit > 1: its
                          // split-K partial sums, added here in slice order; may be qkv)
    const float *q_norm, *k_norm, *rope;
    float eps;
    uint16_t *kcache, *vcache;  // [kv][ctx][64]
    uint32_t T, start, heads, kv, ctx, ksplit;
};

struct AttnPrefillArgs {  // causal GQA attention of T queries at positions start + t
    const float *qkv;     // [T][dim + 2*hdkv] (q already normed + rotated)
    const uint16_t *kcache, *vcache;
    float *out;           // [T][dim]
    float scale;
    uint32_t T, start, heads, kv, ctx;
    // key split (kb_per > 0): grid z = key ranges of kb_per 32-key blocks; range s
    // writes (max, sum, o[64]) of each (query, head) to part[((s T + t) heads + h) 66]
    float *part;
    uint32_t kb_per;
    // nonzero (no key split): grid x = ceil(query tiles / 2), workgroup b takes
    // query tiles n - 1 - b and b
    uint32_t paired;
};

struct AttnMergeSplitArgs { // out[t][h] = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s
    const float *part;
    float *out;
    uint32_t T, heads, nsplit;
    // nullable (small calls): out stored binary16 hi + lo in the blocked layout
    // (logical row t, width heads * 64) with the power-of-two scale of each 128
    // values' largest magnitude at y_bscale[t * (heads * 64 / 128) + k / 128], as the
    // short conv's, for the output projection with no split launch
    uint16_t *y_hi, *y_lo;
    float *y_bscale;
};

struct RouterPrefillArgs {  // logits[t][e] = W_r rmsnorm(x_t)
    const float *x;         // [T][dim]
    const float *norm_w, *w;
    float eps;
    float *logits;          // [T][n_expert]
    uint32_t T, dim, n_expert;
};

struct RouterSplitArgs {    // hi / lo = binary16 split of w * scale (n values)
    const float *w;
    uint16_t *hi, *lo;
    uint32_t n;
    float scale;
};

struct RouterMfmaArgs {     // logits[t][e] = xscale[t] * unscale * sum_k W'[e][k] X'[t][k]
    const uint16_t *x_hi, *x_lo; // [T][K] binary16 split of the FFN input (row-major)
    const float *xscale;         // [T] its row scales
    const uint16_t *w_hi, *w_lo; // [E][K] binary16 split of the router rows times 2^s
    float unscale;               // 2^-s
    float *logits;               // [T][E]
    uint32_t T, K, E;
};

struct RouteGroupArgs {   // per token top-k, then per expert the ordered (token, rank) list
    const float *logits, *bias;  // logits [T][n_expert] (read by k_route_topk)
    uint32_t *sel;        // [T][4] ids
    float *wsel;          // [T][4] weights
    uint32_t *counts;     // [n_expert]
    uint32_t *tok;        // [n_expert][list_stride] activation row (token)
    uint32_t *slot;       // [n_expert][list_stride] slot = t*4 + rank
    uint32_t T, n_expert, n_used, list_stride;
    uint32_t *pos;        // [T*4]: index of slot t*4 + rank in its expert's list
    // the router partials of the preceding reduce (rpart[t][b][e], rss[t][b], b < nparts),
    // handed to the grouped split that routes each token itself; k_route_topk never reads them
    const float *rpart, *rss;
    uint32_t nparts, dim;
    float eps;
};

struct CombinePrefillArgs {  // x[t] += sum_r w[t][r] * D[t*4 + r] (rank order)
    const float *d;          // [T*4][dim]
    const float *wsel;       // [T][4]
    float *x;                // [T][dim]
    uint32_t T, dim, n_used;
};

#define EMBED_INLINE_IDS 64 // forward_token's batch limit
struct EmbedRowsArgs {
    Q6T emb;
    const uint32_t *ids;  // [T]; null: ids_inline (T <= EMBED_INLINE_IDS)
    float *x;             // [T][dim]
    uint32_t T;
    // nullable: workgroup 0 also starts the call's decode state (the host's
    // set_state without a copy): tok = the first id, pos = start, eos = ~0u,
    // n_ids = T, the other fields but gen zero
    DevState *st;
    uint32_t start;
    uint32_t ids_inline[EMBED_INLINE_IDS];
};

// The short-conv mixer of one layer in one launch (k_conv_mixer, k_conv_mixer_r):
// phase A = ConvInprojArgs with one channel per wave (its gated output handed
// on through `flow`, in.y unused); phase B = the output projection y += W g
// (out.m, one row per wave; out.m.src unused), with the router partial sums of
// k_q6_matvec_route in k_conv_mixer_r.  dim / 8 workgroups of 8 waves.
struct ConvMixerArgs {
    ConvInprojArgs in;
    MatvecRouteArgs out;
    unsigned long long *flow; // [dim] tagged entries: gated output bits | tag << 32
    uint32_t phase;           // this launch's phase id in the tags (the layer)
};
