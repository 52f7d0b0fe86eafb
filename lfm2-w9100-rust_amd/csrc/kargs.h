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
    uint32_t pad[7];    // 64 bytes
};

// Where a kernel's input vector comes from.
struct XSrc {
    const float *x;      // residual / activation vector (ignored when embed)
    const float *norm_w; // RMSNorm weight, nullptr = no norm
    float eps;
    uint32_t embed;      // 1: x = dequantized row DevState::tok of `emb`
    Q6T emb;
    float *x_out;        // embed: workgroup 0 writes x here (the residual)
};

struct MatvecArgs {      // y = W x  (mode 0)  or  y += W x  (mode 1)
    Q6T w;
    XSrc src;
    float *y;
    uint32_t in_dim;
    uint32_t mode;
    uint32_t ksplit;     // k_q6_matvec_ks: waves per row (1, 2 or 4)
    uint32_t nbw;        // k_q6_matvec_ks: blocks per wave
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
    const float *logits; // nullptr = dense layer
    const float *bias;
    uint32_t n_expert, n_used;
    uint32_t *sel_out;   // written by one wave: ids[8] then weights[8] (float bits)
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

struct FinalArgs {       // reduce partials; decode step: store, feed back, advance
    const float *partial;
    uint32_t n_partial;
    uint32_t *out_tokens;
    uint32_t advance;
    DevState *st;
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
