/*
 * lfm_oracle.c -- CPU restatement of the reference's LFM2 Q6_K CPU path.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle / CPU baseline).  Nothing in the
 * product may link or call this file.  Build: oracle/Makefile
 * (gcc -O2 -ffp-contract=off -fopenmp, no fast-math).
 *
 * References are to Amidwestnoob/lfm2-w9100-rust (paths relative to its root).
 */
#include "lfm_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;
void oracle_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int oracle_get_threads(void) { return g_threads; }

/* ------------------------------------------------------------------ fp16 */
/* half 2.7.1 f16::to_f32 (used by q6k.rs:56-58): exact IEEE widening. */
float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal half: value = man * 2^-24, exact in f32 */
            float v = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* half 2.7.1 f16::from_f32 (lfm.rs:96-98): IEEE round-to-nearest-even,
 * gradual underflow, overflow to inf, NaN kept quiet with its top payload. */
uint16_t oracle_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mag = x & 0x7fffffffu;
    if (mag > 0x7f800000u) /* NaN */
        return (uint16_t)(sign | 0x7e00u | ((mag >> 13) & 0x3ffu));
    if (mag >= 0x477ff000u) /* rounds to >= 65520 -> inf (65504 is max) */
        return (uint16_t)(sign | 0x7c00u);
    int32_t e = (int32_t)(mag >> 23) - 127; /* unbiased exponent */
    if (e >= -14) {
        /* normal half: keep 10 mantissa bits, RNE on the 13 dropped bits */
        uint32_t m = mag & 0x7fffffu;
        uint32_t keep = m >> 13;
        uint32_t rest = m & 0x1fffu;
        uint32_t out = ((uint32_t)(e + 15) << 10) | keep;
        if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u)))
            out += 1; /* carry may ripple into the exponent: still correct */
        return (uint16_t)(sign | out);
    }
    if (e < -25) /* below half of the smallest subnormal (2^-25): zero */
        return (uint16_t)sign;
    /* subnormal half: value / 2^-24 rounded to an integer, RNE */
    uint32_t m = (mag & 0x7fffffu) | 0x800000u; /* 24-bit significand */
    uint32_t shift = (uint32_t)(-e - 1);        /* e=-15 -> 14 ... e=-25 -> 24 */
    uint32_t keep = m >> shift;
    uint32_t rest = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rest > half || (rest == half && (keep & 1u)))
        keep += 1;
    return (uint16_t)(sign | keep);
}

float oracle_f16_round(float x) { return oracle_f16_to_f32(oracle_f32_to_f16(x)); }

void oracle_f32_to_f16_array(const float *in, uint16_t *out, size_t n)
{
    for (size_t i = 0; i < n; i++)
        out[i] = oracle_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------ Q6_K */
/* q6k.rs:74-146 dequantize_q6k_block_mode(legacy_unsigned = false). */
static void dequant_half(float d, const uint8_t *ql, const uint8_t *qh, const uint8_t *sc,
                         float *y)
{
    for (int l = 0; l < 32; l++) {
        int is = l / 16;
        uint8_t qh_l = qh[l];
        int8_t q1 = (int8_t)((int8_t)(ql[l] & 0x0F) | (int8_t)((qh_l & 0x03) << 4)) - 32;
        int8_t q2 = (int8_t)((int8_t)(ql[l + 32] & 0x0F) | (int8_t)(((qh_l >> 2) & 0x03) << 4)) - 32;
        int8_t q3 = (int8_t)((int8_t)(ql[l] >> 4) | (int8_t)(((qh_l >> 4) & 0x03) << 4)) - 32;
        int8_t q4 = (int8_t)((int8_t)(ql[l + 32] >> 4) | (int8_t)(((qh_l >> 6) & 0x03) << 4)) - 32;
        float s0 = (float)(int8_t)sc[is];
        float s2 = (float)(int8_t)sc[is + 2];
        float s4 = (float)(int8_t)sc[is + 4];
        float s6 = (float)(int8_t)sc[is + 6];
        /* three float multiplies, left to right: (d * s) * q */
        y[l] = d * s0 * (float)q1;
        y[l + 32] = d * s2 * (float)q2;
        y[l + 64] = d * s4 * (float)q3;
        y[l + 96] = d * s6 * (float)q4;
    }
}

void oracle_q6k_dequant_block(const uint8_t *blk, float *out)
{
    float d = oracle_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
    dequant_half(d, blk, blk + 128, blk + 192, out);
    dequant_half(d, blk + 64, blk + 160, blk + 200, out + 128);
}

/* dequant_mirror.rs:10-46: the per-element index formula. */
float oracle_q6k_mirror_elem(const uint8_t *blk, uint32_t k)
{
    uint32_t half = k >> 7, jj = k & 127, sub = jj >> 5, l = jj & 31, is = l >> 4;
    uint32_t ql_idx = half * 64 + l + (sub & 1) * 32;
    uint32_t qh_idx = 128 + half * 32 + l;
    uint32_t sc_idx = 192 + half * 8 + is + 2 * sub;
    uint8_t qlbyte = blk[ql_idx];
    uint32_t nibble = (sub >> 1) ? (uint32_t)(qlbyte >> 4) : (uint32_t)(qlbyte & 0x0F);
    uint32_t field = ((uint32_t)blk[qh_idx] >> (2 * sub)) & 3u;
    int32_t q = (int32_t)(nibble | (field << 4)) - 32;
    int32_t scb = blk[sc_idx];
    int32_t sc = scb >= 128 ? scb - 256 : scb;
    uint16_t dh = (uint16_t)(blk[208] | (blk[209] << 8));
    float d = oracle_f16_to_f32(dh);
    return d * (float)sc * (float)q;
}

/* q6k.rs:150-159 */
void oracle_q6k_dequant_row(const uint8_t *blocks, size_t n, float *out)
{
    for (size_t b = 0; b < n / 256; b++)
        oracle_q6k_dequant_block(blocks + b * 210, out + b * 256);
}

/* q6k.rs:167-183: dequantize a row, f64 dot, round to f32. */
void oracle_q6k_matvec(const uint8_t *w, size_t in_dim, size_t out_dim, const float *x,
                       float *y)
{
    size_t row_bytes = in_dim / 256 * 210;
#pragma omp parallel num_threads(g_threads)
    {
        float *wrow = (float *)malloc(in_dim * sizeof(float));
#pragma omp for schedule(static)
        for (long o = 0; o < (long)out_dim; o++) {
            oracle_q6k_dequant_row(w + (size_t)o * row_bytes, in_dim, wrow);
            double acc = 0.0;
            for (size_t k = 0; k < in_dim; k++)
                acc += (double)wrow[k] * (double)x[k];
            y[o] = (float)acc;
        }
        free(wrow);
    }
}

/* q6k.rs:25-30 */
void oracle_q6k_repack_aligned(const uint8_t *raw, size_t raw_len, uint8_t *out)
{
    for (size_t b = 0; b < raw_len / 210; b++) {
        memcpy(out + b * 212, raw + b * 210, 210);
        out[b * 212 + 210] = 0;
        out[b * 212 + 211] = 0;
    }
}

/* ------------------------------------------------------------------ argmax */
/* main.rs:112-141: eight independent lanes, then lane merge (ties -> lowest
 * index), then the tail.  NaN never wins; all -inf/NaN -> 0. */
uint32_t oracle_argmax(const float *logits, size_t n)
{
    float values[8];
    size_t indices[8];
    for (int i = 0; i < 8; i++) {
        values[i] = -INFINITY;
        indices[i] = 0;
    }
    size_t nchunks = n / 8;
    for (size_t block = 0; block < nchunks; block++)
        for (int lane = 0; lane < 8; lane++) {
            float v = logits[block * 8 + lane];
            if (v > values[lane]) {
                values[lane] = v;
                indices[lane] = block * 8 + lane;
            }
        }
    size_t best = 0;
    float value = -INFINITY;
    for (int lane = 0; lane < 8; lane++)
        if (values[lane] > value || (values[lane] == value && indices[lane] < best)) {
            best = indices[lane];
            value = values[lane];
        }
    size_t offset = nchunks * 8;
    for (size_t i = offset; i < n; i++)
        if (logits[i] > value) {
            best = i;
            value = logits[i];
        }
    return (uint32_t)best;
}

/* main.rs:289-298: the scalar statement the lane form must equal. */
uint32_t oracle_argmax_scalar(const float *xs, size_t n)
{
    uint32_t best = 0;
    float value = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (xs[i] > value) {
            best = (uint32_t)i;
            value = xs[i];
        }
    return best;
}

/* ------------------------------------------------------------------ route */
/* lfm.rs:613-637: sigmoid probabilities, score = p + bias, stable descending
 * sort (ties keep the lower expert id first), weights p[sel] / max(sum, 2^-14). */
void oracle_route(const float *router, const float *bias, uint32_t n_expert, uint32_t n_used,
                  uint32_t *sel, float *wsel, float *probs_out)
{
    float probs[256];
    float score[256];
    uint32_t order[256];
    for (uint32_t e = 0; e < n_expert; e++) {
        float lg = router[e];
        probs[e] = 1.0f / (1.0f + expf(-lg));
        score[e] = probs[e] + bias[e];
        order[e] = e;
    }
    /* stable insertion sort, descending by score */
    for (uint32_t i = 1; i < n_expert; i++) {
        uint32_t cur = order[i];
        int j = (int)i - 1;
        while (j >= 0 && score[order[j]] < score[cur]) {
            order[j + 1] = order[j];
            j--;
        }
        order[j + 1] = cur;
    }
    float wsum = 0.0f;
    for (uint32_t r = 0; r < n_used; r++) {
        sel[r] = order[r];
        wsel[r] = probs[order[r]];
        wsum += probs[order[r]];
    }
    if (wsum < 6.103515625e-5f)
        wsum = 6.103515625e-5f;
    for (uint32_t r = 0; r < n_used; r++)
        wsel[r] /= wsum;
    if (probs_out)
        for (uint32_t e = 0; e < n_expert; e++)
            probs_out[e] = score[e];
}

/* f32::powi as lowered for a run-time exponent (compiler-rt __powisf2):
 * square-and-multiply, r starting at 1. */
float oracle_powi(float a, int b)
{
    int recip = b < 0;
    float r = 1.0f;
    for (;;) {
        if (b & 1)
            r *= a;
        b /= 2;
        if (b == 0)
            break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

/* ------------------------------------------------------------------ engine */
typedef struct tensor {
    char name[96];
    uint32_t type;
    uint64_t ne[4];
    uint32_t nd;
    uint8_t *data;
    size_t nbytes;
    float *f32; /* dequantized / copied f32 for non-3D tensors */
} tensor;

struct oracle_engine {
    oracle_hparams hp;
    uint32_t ctx;
    int kv_f16;
    tensor *t;
    size_t nt, cap;
    float *conv[ORACLE_MAX_LAYERS];   /* [ch][slot], cache_len slots */
    float *keys[ORACLE_MAX_LAYERS];   /* [t][kh][d] */
    float *values[ORACLE_MAX_LAYERS]; /* [kh][d][t] */
    uint32_t route_ids[ORACLE_MAX_LAYERS][8];
    float route_w[ORACLE_MAX_LAYERS][8];
    float route_scores[ORACLE_MAX_LAYERS][256];
};

oracle_engine *oracle_engine_create(const oracle_hparams *hp, uint32_t ctx, int kv_f16)
{
    if (!hp || hp->n_layers > ORACLE_MAX_LAYERS || hp->n_expert > 256 || hp->n_used > 8)
        return NULL;
    oracle_engine *e = (oracle_engine *)calloc(1, sizeof(*e));
    e->hp = *hp;
    e->ctx = ctx;
    e->kv_f16 = kv_f16;
    return e;
}

static void free_state(oracle_engine *e)
{
    for (int l = 0; l < ORACLE_MAX_LAYERS; l++) {
        free(e->conv[l]);
        free(e->keys[l]);
        free(e->values[l]);
        e->conv[l] = e->keys[l] = e->values[l] = NULL;
    }
}

void oracle_engine_destroy(oracle_engine *e)
{
    if (!e)
        return;
    for (size_t i = 0; i < e->nt; i++) {
        free(e->t[i].data);
        free(e->t[i].f32);
    }
    free(e->t);
    free_state(e);
    free(e);
}

void oracle_reset(oracle_engine *e) { free_state(e); }

static tensor *find(const oracle_engine *e, const char *name)
{
    for (size_t i = 0; i < e->nt; i++)
        if (strcmp(e->t[i].name, name) == 0)
            return &e->t[i];
    return NULL;
}

int oracle_engine_set_tensor(oracle_engine *e, const char *name, uint32_t type,
                             const uint64_t *ne, uint32_t nd, const void *data, size_t nbytes)
{
    if (!e || !name || strlen(name) >= 96 || nd < 1 || nd > 4)
        return -1;
    tensor *t = find(e, name);
    if (!t) {
        if (e->nt == e->cap) {
            e->cap = e->cap ? e->cap * 2 : 64;
            e->t = (tensor *)realloc(e->t, e->cap * sizeof(tensor));
        }
        t = &e->t[e->nt++];
        memset(t, 0, sizeof(*t));
        strcpy(t->name, name);
    }
    free(t->data);
    free(t->f32);
    t->f32 = NULL;
    t->type = type;
    t->nd = nd;
    for (uint32_t i = 0; i < 4; i++)
        t->ne[i] = i < nd ? ne[i] : 1;
    t->data = (uint8_t *)malloc(nbytes ? nbytes : 1);
    memcpy(t->data, data, nbytes);
    t->nbytes = nbytes;
    return 0;
}

/* lfm.rs:165-179: dequantize every non-3D tensor once. */
int oracle_engine_finalize(oracle_engine *e)
{
    for (size_t i = 0; i < e->nt; i++) {
        tensor *t = &e->t[i];
        if (t->nd == 3 || t->f32)
            continue;
        size_t n = (size_t)(t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]);
        t->f32 = (float *)malloc(n * sizeof(float));
        if (t->type == ORACLE_GGML_F32) {
            memcpy(t->f32, t->data, n * sizeof(float));
        } else if (t->type == ORACLE_GGML_Q6_K) {
            size_t nblk = n / 256;
#pragma omp parallel for num_threads(g_threads) schedule(static)
            for (long b = 0; b < (long)nblk; b++)
                oracle_q6k_dequant_block(t->data + (size_t)b * 210, t->f32 + (size_t)b * 256);
        } else {
            return -2;
        }
    }
    return 0;
}

static const float *f32_of(const oracle_engine *e, const char *name)
{
    tensor *t = find(e, name);
    return t ? t->f32 : NULL;
}

/* lfm.rs:205-228: out[o + j*out] = f32-sequential dot over k. */
static int mul_mat_weight(const oracle_engine *e, const char *wname, size_t in_dim,
                          size_t out_dim, const float *x, size_t n, float *out)
{
    const float *w = f32_of(e, wname);
    if (!w)
        return -3;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (long o = 0; o < (long)out_dim; o++) {
        const float *row = w + (size_t)o * in_dim;
        for (size_t j = 0; j < n; j++) {
            float acc = 0.0f;
            for (size_t k = 0; k < in_dim; k++)
                acc += row[k] * x[k + j * in_dim];
            out[o + j * out_dim] = acc;
        }
    }
    return 0;
}

/* lfm.rs:698-725: expert slice of a 3D Q6_K tensor, re-dequantized per row. */
static int mul_mat_expert(const oracle_engine *e, const char *wname, size_t expert,
                          size_t in_dim, size_t out_dim, const float *x, float *out)
{
    tensor *t = find(e, wname);
    if (!t || t->type != ORACLE_GGML_Q6_K)
        return -3;
    size_t row_bytes = in_dim / 256 * 210;
    size_t base = expert * out_dim * row_bytes;
#pragma omp parallel num_threads(g_threads)
    {
        float *wrow = (float *)malloc(in_dim * sizeof(float));
#pragma omp for schedule(static)
        for (long o = 0; o < (long)out_dim; o++) {
            oracle_q6k_dequant_row(t->data + base + (size_t)o * row_bytes, in_dim, wrow);
            float acc = 0.0f;
            for (size_t k = 0; k < in_dim; k++)
                acc += wrow[k] * x[k];
            out[o] = acc;
        }
        free(wrow);
    }
    return 0;
}

/* lfm.rs:231-244 */
static void rms_norm(const oracle_engine *e, const float *x, const float *scale, size_t n,
                     float *out)
{
    size_t dim = e->hp.dim;
    for (size_t j = 0; j < n; j++) {
        float ss = 0.0f;
        for (size_t k = 0; k < dim; k++) {
            float v = x[k + j * dim];
            ss += v * v;
        }
        float inv = 1.0f / sqrtf(ss / (float)dim + e->hp.eps);
        for (size_t k = 0; k < dim; k++)
            out[k + j * dim] = x[k + j * dim] * inv * scale[k];
    }
}

/* lfm.rs:248-267: NEOX RoPE, pairs (p, p + hd/2). */
static void rope_neox(const oracle_engine *e, float *q, size_t heads, size_t n,
                      const int64_t *positions)
{
    size_t hd = e->hp.head_dim;
    size_t dim_all = hd * heads;
    float tscale = powf(e->hp.rope_theta, -2.0f / (float)hd);
    for (size_t j = 0; j < n; j++) {
        float pos = (float)positions[j];
        for (size_t p = 0; p < hd / 2; p++) {
            float theta = pos * oracle_powi(tscale, (int)p);
            float s = sinf(theta), c = cosf(theta);
            for (size_t h = 0; h < heads; h++) {
                size_t i0 = p + h * hd + j * dim_all;
                size_t i1 = p + hd / 2 + h * hd + j * dim_all;
                float x0 = q[i0], x1 = q[i1];
                q[i0] = x0 * c - x1 * s;
                q[i1] = x0 * s + x1 * c;
            }
        }
    }
}

/* lfm.rs:270-286: q *= inv * scale[k]. */
static void norm_head_dim(const oracle_engine *e, float *q, const float *scale, size_t heads,
                          size_t n)
{
    size_t hd = e->hp.head_dim;
    size_t dim_all = hd * heads;
    for (size_t h = 0; h < heads; h++)
        for (size_t j = 0; j < n; j++) {
            float ss = 0.0f;
            for (size_t k = 0; k < hd; k++) {
                float v = q[k + h * hd + j * dim_all];
                ss += v * v;
            }
            float inv = 1.0f / sqrtf(ss / (float)hd + e->hp.eps);
            for (size_t k = 0; k < hd; k++)
                q[k + h * hd + j * dim_all] *= inv * scale[k];
        }
}

static void ensure_kv(oracle_engine *e, uint32_t l, size_t kv)
{
    if (!e->keys[l]) {
        size_t n = e->hp.head_dim * kv * e->ctx;
        e->keys[l] = (float *)calloc(n, sizeof(float));
        e->values[l] = (float *)calloc(n, sizeof(float));
    }
}

static void ensure_conv(oracle_engine *e, uint32_t l)
{
    if (!e->conv[l])
        e->conv[l] = (float *)calloc((size_t)e->hp.dim * (e->hp.conv_l_cache - 1), sizeof(float));
}

#define NAME(buf, l, suffix) (snprintf((buf), sizeof(buf), "blk.%u." suffix, (unsigned)(l)), (buf))

/* lfm.rs:337-449: attention mixer on h[dim*n]; adds the projection into x. */
static int attention_layer(oracle_engine *e, uint32_t l, const float *h, float *x, size_t n,
                           int64_t start_pos)
{
    const oracle_hparams *hp = &e->hp;
    size_t dim = hp->dim, hd = hp->head_dim, kv = hp->kv_heads[l], heads = hp->heads;
    size_t hdkv = hd * kv, ctx = e->ctx;
    char nm[128];
    if (start_pos < 0 || (size_t)start_pos + n > ctx)
        return -4;
    float *q = (float *)malloc(dim * n * sizeof(float));
    float *k = (float *)malloc(hdkv * n * sizeof(float));
    float *v = (float *)malloc(hdkv * n * sizeof(float));
    int rc = 0;
    rc |= mul_mat_weight(e, NAME(nm, l, "attn_q.weight"), dim, dim, h, n, q);
    rc |= mul_mat_weight(e, NAME(nm, l, "attn_k.weight"), dim, hdkv, h, n, k);
    rc |= mul_mat_weight(e, NAME(nm, l, "attn_v.weight"), dim, hdkv, h, n, v);
    const float *qn = f32_of(e, NAME(nm, l, "attn_q_norm.weight"));
    const float *kn = f32_of(e, NAME(nm, l, "attn_k_norm.weight"));
    if (rc || !qn || !kn) {
        free(q), free(k), free(v);
        return -3;
    }
    norm_head_dim(e, q, qn, heads, n);
    norm_head_dim(e, k, kn, kv, n);
    int64_t *positions = (int64_t *)malloc(n * sizeof(int64_t));
    for (size_t i = 0; i < n; i++)
        positions[i] = start_pos + (int64_t)i;
    rope_neox(e, q, heads, n, positions);
    rope_neox(e, k, kv, n, positions);
    free(positions);

    ensure_kv(e, l, kv);
    float *keys = e->keys[l], *values = e->values[l];
    for (size_t j = 0; j < n; j++) {
        size_t p = (size_t)start_pos + j;
        for (size_t kh = 0; kh < kv; kh++)
            for (size_t d = 0; d < hd; d++) {
                float kk = k[(kh * hd + d) + j * hdkv];
                float vv = v[(kh * hd + d) + j * hdkv];
                keys[d + kh * hd + p * hdkv] = e->kv_f16 ? oracle_f16_round(kk) : kk;
                values[p + d * ctx + kh * (ctx * hd)] = e->kv_f16 ? oracle_f16_round(vv) : vv;
            }
    }

    float scale = 1.0f / sqrtf((float)hd);
    float *a = (float *)malloc(dim * n * sizeof(float));
    for (size_t j = 0; j < n; j++) {
        size_t p = (size_t)start_pos + j;
#pragma omp parallel num_threads(g_threads)
        {
            float *s = (float *)malloc((p + 1) * sizeof(float));
#pragma omp for schedule(static)
            for (long hh = 0; hh < (long)heads; hh++) {
                size_t kh = (size_t)hh * kv / heads;
                float m = -INFINITY;
                for (size_t t = 0; t <= p; t++) {
                    double acc = 0.0;
                    for (size_t d = 0; d < hd; d++)
                        acc += (double)q[(hh * hd + d) + j * dim] *
                               (double)keys[d + kh * hd + t * hdkv];
                    float sc = (float)acc * scale;
                    s[t] = sc;
                    if (sc > m)
                        m = sc;
                }
                double sum = 0.0;
                for (size_t t = 0; t <= p; t++) {
                    double ev = exp((double)(s[t] - m));
                    s[t] = (float)ev;
                    sum += ev;
                }
                for (size_t t = 0; t <= p; t++)
                    s[t] = (float)((double)s[t] / sum);
                for (size_t d = 0; d < hd; d++) {
                    double acc = 0.0;
                    for (size_t t = 0; t <= p; t++)
                        acc += (double)s[t] * (double)values[t + d * ctx + kh * (ctx * hd)];
                    a[(hh * hd + d) + j * dim] = (float)acc;
                }
            }
            free(s);
        }
    }
    float *ax = (float *)malloc(dim * n * sizeof(float));
    rc = mul_mat_weight(e, NAME(nm, l, "attn_output.weight"), dim, dim, a, n, ax);
    if (!rc)
        for (size_t i = 0; i < dim * n; i++)
            x[i] += ax[i];
    free(q), free(k), free(v), free(a), free(ax);
    return rc;
}

/* lfm.rs:450-533: gated short convolution; adds out_proj into x. */
static int shortconv_layer(oracle_engine *e, uint32_t l, const float *h, float *x, size_t n)
{
    const oracle_hparams *hp = &e->hp;
    size_t dim = hp->dim, conv_l = hp->conv_l_cache, cache_len = conv_l - 1;
    char nm[128];
    float *bcx = (float *)malloc(3 * dim * n * sizeof(float));
    int rc = mul_mat_weight(e, NAME(nm, l, "shortconv.in_proj.weight"), dim, 3 * dim, h, n, bcx);
    const float *cw = f32_of(e, NAME(nm, l, "shortconv.conv.weight"));
    if (rc || !cw) {
        free(bcx);
        return -3;
    }
    float *bx = (float *)malloc(n * dim * sizeof(float));
    for (size_t t = 0; t < n; t++)
        for (size_t ch = 0; ch < dim; ch++) {
            float b = bcx[ch + t * (3 * dim)];
            float xx = bcx[2 * dim + ch + t * (3 * dim)];
            bx[t + ch * n] = b * xx;
        }
    ensure_conv(e, l);
    float *cache = e->conv[l];
    size_t cl = cache_len + n;
    float *ci = (float *)malloc(cl * dim * sizeof(float));
    for (size_t ch = 0; ch < dim; ch++) {
        for (size_t t2 = 0; t2 < cache_len; t2++)
            ci[t2 + ch * cl] = cache[t2 + ch * cache_len];
        for (size_t t2 = 0; t2 < n; t2++)
            ci[cache_len + t2 + ch * cl] = bx[t2 + ch * n];
    }
    for (size_t ch = 0; ch < dim; ch++)
        for (size_t t2 = 0; t2 < cache_len; t2++)
            cache[t2 + ch * cache_len] = ci[n + t2 + ch * cl];
    float *gated = (float *)malloc(dim * n * sizeof(float));
    for (size_t t = 0; t < n; t++)
        for (size_t ch = 0; ch < dim; ch++) {
            float acc = 0.0f;
            for (size_t kk = 0; kk < conv_l; kk++)
                acc += ci[(t + kk) + ch * cl] * cw[kk + ch * conv_l];
            float cc = bcx[dim + ch + t * (3 * dim)];
            gated[ch + t * dim] = cc * acc;
        }
    float *proj = (float *)malloc(dim * n * sizeof(float));
    rc = mul_mat_weight(e, NAME(nm, l, "shortconv.out_proj.weight"), dim, dim, gated, n, proj);
    if (!rc)
        for (size_t i = 0; i < dim * n; i++)
            x[i] += proj[i];
    free(bcx), free(bx), free(ci), free(gated), free(proj);
    return rc;
}

int oracle_run_mixer(oracle_engine *e, uint32_t l, float *x, uint32_t n, int64_t start_pos)
{
    if (!e || l >= e->hp.n_layers || n == 0)
        return -1;
    char nm[128];
    size_t dim = e->hp.dim;
    const float *attn_norm = f32_of(e, NAME(nm, l, "attn_norm.weight"));
    if (!attn_norm)
        return -3;
    float *h = (float *)malloc(dim * n * sizeof(float));
    rms_norm(e, x, attn_norm, n, h);
    int rc = e->hp.kv_heads[l] > 0 ? attention_layer(e, l, h, x, n, start_pos)
                                   : shortconv_layer(e, l, h, x, n);
    free(h);
    return rc;
}

/* lfm.rs:599-607: router logits [nf][n_expert] of normed columns fnorm (the
 * f32 sequential ffn_gate_inp matmul), and the layer's bias vector. */
static int router_logits(oracle_engine *e, uint32_t l, const float *fnorm, size_t nf,
                         float *router, const float **bias)
{
    char nm[128];
    int rc = mul_mat_weight(e, NAME(nm, l, "ffn_gate_inp.weight"), e->hp.dim, e->hp.n_expert,
                            fnorm, nf, router);
    tensor *bt = find(e, NAME(nm, l, "exp_probs_b.bias"));
    if (rc || !bt || !bt->f32)
        return -3;
    *bias = bt->f32;
    return 0;
}

/* lfm.rs:539-670 on columns [f_off, f_off + nf) of x. */
static int ffn_cols(oracle_engine *e, uint32_t l, float *x, size_t f_off, size_t nf)
{
    const oracle_hparams *hp = &e->hp;
    size_t dim = hp->dim;
    char nm[128], nm2[128], nm3[128];
    const float *ffn_norm = f32_of(e, NAME(nm, l, "ffn_norm.weight"));
    if (!ffn_norm)
        return -3;
    float *fnorm = (float *)malloc(dim * nf * sizeof(float));
    rms_norm(e, x + f_off * dim, ffn_norm, nf, fnorm);
    int rc = 0;
    if (l < hp->dense_lead) {
        size_t ff = hp->n_ff;
        float *gate = (float *)malloc(ff * nf * sizeof(float));
        float *up = (float *)malloc(ff * nf * sizeof(float));
        float *out = (float *)malloc(dim * nf * sizeof(float));
        rc |= mul_mat_weight(e, NAME(nm, l, "ffn_gate.weight"), dim, ff, fnorm, nf, gate);
        rc |= mul_mat_weight(e, NAME(nm, l, "ffn_up.weight"), dim, ff, fnorm, nf, up);
        for (size_t i = 0; i < ff * nf && !rc; i++) {
            float g = gate[i];
            gate[i] = g / (1.0f + expf(-g)) * up[i];
        }
        if (!rc)
            rc |= mul_mat_weight(e, NAME(nm, l, "ffn_down.weight"), ff, dim, gate, nf, out);
        if (!rc)
            for (size_t j = 0; j < nf; j++)
                for (size_t k = 0; k < dim; k++)
                    x[k + (f_off + j) * dim] += out[k + j * dim];
        free(gate), free(up), free(out);
    } else {
        size_t ne = hp->n_expert, nu = hp->n_used, eff = hp->expert_ff;
        float *router = (float *)malloc(ne * nf * sizeof(float));
        const float *bias = NULL;
        if (router_logits(e, l, fnorm, nf, router, &bias)) {
            free(router), free(fnorm);
            return -3;
        }
        NAME(nm, l, "ffn_gate_exps.weight");
        NAME(nm2, l, "ffn_up_exps.weight");
        NAME(nm3, l, "ffn_down_exps.weight");
        float *gate_e = (float *)malloc(eff * sizeof(float));
        float *up_e = (float *)malloc(eff * sizeof(float));
        float *down_e = (float *)malloc(dim * sizeof(float));
        float *acc = (float *)malloc(dim * sizeof(float));
        for (size_t j = 0; j < nf && !rc; j++) {
            uint32_t sel[8];
            float wsel[8];
            oracle_route(router + j * ne, bias, (uint32_t)ne, (uint32_t)nu, sel, wsel,
                         e->route_scores[l]);
            for (size_t r = 0; r < nu; r++) {
                e->route_ids[l][r] = sel[r];
                e->route_w[l][r] = wsel[r];
            }
            const float *fcol = fnorm + j * dim;
            for (size_t k = 0; k < dim; k++)
                acc[k] = 0.0f;
            for (size_t r = 0; r < nu && !rc; r++) {
                size_t ex = sel[r];
                rc |= mul_mat_expert(e, nm, ex, dim, eff, fcol, gate_e);
                rc |= mul_mat_expert(e, nm2, ex, dim, eff, fcol, up_e);
                for (size_t i = 0; i < eff; i++) {
                    float g = gate_e[i];
                    gate_e[i] = g / (1.0f + expf(-g)) * up_e[i];
                }
                rc |= mul_mat_expert(e, nm3, ex, eff, dim, gate_e, down_e);
                for (size_t k = 0; k < dim; k++)
                    acc[k] += down_e[k] * wsel[r];
            }
            for (size_t k = 0; k < dim; k++)
                x[k + (f_off + j) * dim] += acc[k];
        }
        free(router), free(gate_e), free(up_e), free(down_e), free(acc);
    }
    free(fnorm);
    return rc;
}

int oracle_run_ffn(oracle_engine *e, uint32_t l, float *x, uint32_t n)
{
    if (!e || l >= e->hp.n_layers || n == 0)
        return -1;
    return ffn_cols(e, l, x, 0, n);
}

/* The routing step of ffn_cols alone (lfm.rs:599-637): RMSNorm of x with the
 * layer's ffn_norm, router logits, selection and weights; x is not changed. */
int oracle_route_layer(oracle_engine *e, uint32_t l, const float *x, uint32_t *ids, float *w,
                       float *scores, float *logits)
{
    if (!e || l >= e->hp.n_layers || l < e->hp.dense_lead || !x || !ids || !w)
        return -1;
    char nm[128];
    const float *ffn_norm = f32_of(e, NAME(nm, l, "ffn_norm.weight"));
    if (!ffn_norm)
        return -3;
    size_t dim = e->hp.dim, ne = e->hp.n_expert;
    float *fnorm = (float *)malloc(dim * sizeof(float));
    float *router = (float *)malloc(ne * sizeof(float));
    rms_norm(e, x, ffn_norm, 1, fnorm);
    const float *bias = NULL;
    int rc = router_logits(e, l, fnorm, 1, router, &bias);
    if (!rc) {
        oracle_route(router, bias, (uint32_t)ne, e->hp.n_used, ids, w, scores);
        if (logits)
            memcpy(logits, router, ne * sizeof(float));
    }
    free(fnorm), free(router);
    return rc;
}

int oracle_embed(oracle_engine *e, uint32_t token, float *out)
{
    const float *emb = f32_of(e, "token_embd.weight");
    if (!emb || token >= e->hp.vocab)
        return -3;
    memcpy(out, emb + (size_t)token * e->hp.dim, e->hp.dim * sizeof(float));
    return 0;
}

/* lfm.rs:676-693 */
int oracle_head(oracle_engine *e, const float *xl, float *logits)
{
    size_t dim = e->hp.dim;
    const float *onorm = f32_of(e, "token_embd_norm.weight");
    if (!onorm)
        return -3;
    float *xnorm = (float *)malloc(dim * sizeof(float));
    float ss = 0.0f;
    for (size_t k = 0; k < dim; k++)
        ss += xl[k] * xl[k];
    float inv = 1.0f / sqrtf(ss / (float)dim + e->hp.eps);
    for (size_t k = 0; k < dim; k++)
        xnorm[k] = xl[k] * inv * onorm[k];
    int rc = mul_mat_weight(e, "token_embd.weight", dim, e->hp.vocab, xnorm, 1, logits);
    free(xnorm);
    return rc;
}

/* lfm.rs:290-694 */
int oracle_forward(oracle_engine *e, const uint32_t *ids, uint32_t n, int64_t start_pos,
                   float *logits)
{
    if (!e || n == 0 || start_pos < 0 || (uint64_t)start_pos + n > e->ctx)
        return -1;
    size_t dim = e->hp.dim;
    for (uint32_t j = 0; j < n; j++)
        if (ids[j] >= e->hp.vocab)
            return -1;
    float *x = (float *)malloc(dim * n * sizeof(float));
    int rc = 0;
    for (uint32_t j = 0; j < n && !rc; j++)
        rc = oracle_embed(e, ids[j], x + (size_t)j * dim);
    for (uint32_t l = 0; l < e->hp.n_layers && !rc; l++) {
        rc = oracle_run_mixer(e, l, x, n, start_pos);
        if (rc)
            break;
        size_t nf = (l == e->hp.n_layers - 1) ? 1 : n;
        size_t f_off = nf == 1 ? n - 1 : 0;
        rc = ffn_cols(e, l, x, f_off, nf);
    }
    if (!rc)
        rc = oracle_head(e, x + (size_t)(n - 1) * dim, logits);
    free(x);
    return rc;
}

size_t oracle_state_bytes(const oracle_engine *e, uint32_t valid)
{
    size_t total = 0;
    for (uint32_t l = 0; l < e->hp.n_layers; l++) {
        uint32_t kv = e->hp.kv_heads[l];
        if (kv > 0)
            total += 2 * (size_t)e->hp.head_dim * kv * valid * 4;
        else
            total += (size_t)e->hp.dim * (e->hp.conv_l_cache - 1) * 4;
    }
    return total;
}

/* resident_graph.rs:572-602 byte order (K [t][kh][d] then V [t][kh][d]). */
int oracle_snapshot(const oracle_engine *e, uint32_t valid, uint8_t *buf, size_t cap)
{
    if (valid > e->ctx || cap < oracle_state_bytes(e, valid))
        return -1;
    float *out = (float *)buf;
    size_t o = 0, hd = e->hp.head_dim, ctx = e->ctx;
    for (uint32_t l = 0; l < e->hp.n_layers; l++) {
        size_t kv = e->hp.kv_heads[l];
        if (kv > 0) {
            for (size_t t = 0; t < valid; t++)
                for (size_t kh = 0; kh < kv; kh++)
                    for (size_t d = 0; d < hd; d++)
                        out[o++] = e->keys[l] ? e->keys[l][d + kh * hd + t * hd * kv] : 0.0f;
            for (size_t t = 0; t < valid; t++)
                for (size_t kh = 0; kh < kv; kh++)
                    for (size_t d = 0; d < hd; d++)
                        out[o++] = e->values[l] ? e->values[l][t + d * ctx + kh * ctx * hd] : 0.0f;
        } else {
            size_t cn = (size_t)e->hp.dim * (e->hp.conv_l_cache - 1);
            for (size_t i = 0; i < cn; i++)
                out[o++] = e->conv[l] ? e->conv[l][i] : 0.0f;
        }
    }
    return 0;
}

int oracle_restore(oracle_engine *e, uint32_t valid, const uint8_t *buf, size_t len)
{
    if (valid > e->ctx || len != oracle_state_bytes(e, valid))
        return -1;
    const float *in = (const float *)buf;
    size_t o = 0, hd = e->hp.head_dim, ctx = e->ctx;
    for (uint32_t l = 0; l < e->hp.n_layers; l++) {
        size_t kv = e->hp.kv_heads[l];
        if (kv > 0) {
            ensure_kv(e, l, kv);
            for (size_t t = 0; t < valid; t++)
                for (size_t kh = 0; kh < kv; kh++)
                    for (size_t d = 0; d < hd; d++)
                        e->keys[l][d + kh * hd + t * hd * kv] = in[o++];
            for (size_t t = 0; t < valid; t++)
                for (size_t kh = 0; kh < kv; kh++)
                    for (size_t d = 0; d < hd; d++)
                        e->values[l][t + d * ctx + kh * ctx * hd] = in[o++];
        } else {
            ensure_conv(e, l);
            size_t cn = (size_t)e->hp.dim * (e->hp.conv_l_cache - 1);
            for (size_t i = 0; i < cn; i++)
                e->conv[l][i] = in[o++];
        }
    }
    return 0;
}

int oracle_last_route(const oracle_engine *e, uint32_t l, uint32_t *ids, float *w, float *scores)
{
    if (!e || l >= e->hp.n_layers)
        return -1;
    for (uint32_t r = 0; r < e->hp.n_used; r++) {
        ids[r] = e->route_ids[l][r];
        w[r] = e->route_w[l][r];
    }
    if (scores)
        memcpy(scores, e->route_scores[l], e->hp.n_expert * sizeof(float));
    return 0;
}
