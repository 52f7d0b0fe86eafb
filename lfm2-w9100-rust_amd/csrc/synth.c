/*
 * synth.c -- seeded synthetic LFM2.5-8B-A1B-shaped Q6_K model generator and
 * host binary16 helpers.  Every tensor is a pure function of (seed, tensor
 * name, element index): counter-based SplitMix64 streams (Steele, Lea &
 * Flood 2014) and Box-Muller normals in f64, so any host produces identical
 * bytes regardless of the thread count.
 *
 * Tensor names/shapes follow the reference's model (engine/src/lfm.rs:330-669,
 * resident_graph.rs:237-503).  Distributions:
 *   Q6_K weights : ql/qh uniform bytes, int8 scales uniform in [-32, 31]
 *                  (full_scales: uniform in [-127, 127] with one sub-block of
 *                  each super-block at -128, the form ggml's Q6_K quantizer
 *                  writes: the largest-magnitude scale maps to -128),
 *                  d = binary16(N(0, d_sigma))
 *   norms        : 1 + N(0, norm_sigma)           router: N(0, router_sigma)
 *   expert bias  : N(0, bias_sigma) (zeros if 0)  conv  : N(0, conv_sigma)
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/lfm_hip.h"

/* ---------------------------------------------------------------- binary16 */
float lfm_f16_to_f32(uint16_t h)
{
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    float out;
    if (e == 0) {
        out = ldexpf((float)m, -24); /* zero or subnormal: m * 2^-24, exact */
        uint32_t b;
        memcpy(&b, &out, 4);
        b |= s;
        memcpy(&out, &b, 4);
        return out;
    }
    uint32_t b = e == 31 ? (s | 0x7f800000u | (m << 13)) : (s | ((e + 112u) << 23) | (m << 13));
    memcpy(&out, &b, 4);
    return out;
}

uint16_t lfm_f32_to_f16(float f)
{
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint16_t s = (uint16_t)((b >> 16) & 0x8000u);
    const uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) /* NaN: quiet, top payload bits kept */
        return (uint16_t)(s | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) /* >= 65520 rounds to infinity */
        return (uint16_t)(s | 0x7c00u);
    if (a >= 0x38800000u) { /* normal result (>= 2^-14) */
        /* add the rounding bias (0xfff + lsb) then drop 13 bits: RNE */
        const uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
        return (uint16_t)(s | ((r - 0x38000000u) >> 13));
    }
    if (a < 0x33000001u) /* <= 2^-25 (half of the smallest subnormal, ties to 0) */
        return s;
    /* subnormal result: significand shifted right by (126 - exp) with RNE */
    const uint32_t e = a >> 23;
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;
    const uint32_t sh = 126u - e; /* 14 .. 24 */
    uint32_t q = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), halfway = 1u << (sh - 1u);
    if (rem > halfway || (rem == halfway && (q & 1u)))
        q++;
    return (uint16_t)(s | q);
}

/* ---------------------------------------------------------------- streams */
static uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t sm_next(uint64_t *s)
{
    *s += 0x9E3779B97F4A7C15ull;
    return mix64(*s);
}

static uint64_t stream_seed(uint64_t seed, const char *name)
{
    uint64_t h = 0xcbf29ce484222325ull; /* FNV-1a 64 */
    for (const unsigned char *p = (const unsigned char *)name; *p; ++p) {
        h ^= *p;
        h *= 0x100000001b3ull;
    }
    return mix64(h ^ mix64(seed));
}

/* Box-Muller pair from two 53-bit uniforms: u1 in (0, 1], u2 in [0, 1). */
static void normal_pair(uint64_t *s, double *z0, double *z1)
{
    const double u1 = (double)((sm_next(s) >> 11) + 1) * 0x1.0p-53;
    const double u2 = (double)(sm_next(s) >> 11) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586476925286766559 * u2;
    *z0 = r * cos(t);
    *z1 = r * sin(t);
}

static void q6k_block(uint64_t tseed, uint64_t b, float d_sigma, int full, uint8_t *out)
{
    uint64_t s = tseed + (b + 1) * 0xD1B54A32D192ED03ull;
    for (int i = 0; i < 24; ++i) {
        const uint64_t v = sm_next(&s);
        for (int k = 0; k < 8; ++k)
            out[i * 8 + k] = (uint8_t)(v >> (8 * k));
    }
    for (int i = 0; i < 2; ++i) {
        const uint64_t v = sm_next(&s);
        for (int k = 0; k < 8; ++k) {
            const int byte = (int)((v >> (8 * k)) & 255u);
            out[192 + i * 8 + k] = (uint8_t)(int8_t)(full ? byte % 255 - 127 : (byte & 63) - 32);
        }
    }
    if (full)
        out[192 + (sm_next(&s) & 15u)] = (uint8_t)(int8_t)-128;
    double z0, z1;
    normal_pair(&s, &z0, &z1);
    const uint16_t d = lfm_f32_to_f16((float)(d_sigma * z0));
    out[208] = (uint8_t)(d & 0xff);
    out[209] = (uint8_t)(d >> 8);
}

typedef struct job {
    int kind; /* 0 q6k, 1 normal, 2 q6k with full-range scales */
    uint64_t tseed, begin, end;
    float a, b; /* q6k: d_sigma; normal: mean, sigma */
    void *out;
} job;

static void run_job(job *j)
{
    if (j->kind == 0 || j->kind == 2) {
        for (uint64_t b = j->begin; b < j->end; ++b)
            q6k_block(j->tseed, b, j->a, j->kind == 2, (uint8_t *)j->out + b * 210);
    } else {
        float *o = (float *)j->out;
        for (uint64_t k = j->begin; k < j->end; ++k) { /* k = pair index */
            uint64_t s = j->tseed + (k + 1) * 0xD1B54A32D192ED03ull;
            double z0, z1;
            normal_pair(&s, &z0, &z1);
            o[2 * k] = (float)(j->a + j->b * z0);
            o[2 * k + 1] = (float)(j->a + j->b * z1); /* odd tail: lfm_synth_normal_f32 */
        }
    }
}

static void *job_thread(void *p)
{
    run_job((job *)p);
    return NULL;
}

static void run_parallel(job proto, uint64_t n, int threads)
{
    if (threads < 1)
        threads = 1;
    if (threads > 64)
        threads = 64;
    if ((uint64_t)threads > n)
        threads = n ? (int)n : 1;
    if (threads == 1) {
        proto.begin = 0;
        proto.end = n;
        run_job(&proto);
        return;
    }
    job jobs[64];
    pthread_t tid[64];
    for (int t = 0; t < threads; ++t) {
        jobs[t] = proto;
        jobs[t].begin = n * (uint64_t)t / (uint64_t)threads;
        jobs[t].end = n * (uint64_t)(t + 1) / (uint64_t)threads;
        pthread_create(&tid[t], NULL, job_thread, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t)
        pthread_join(tid[t], NULL);
}

int lfm_synth_q6k_blocks_ex(uint64_t seed, const char *stream, uint64_t nblocks, float d_sigma,
                            int full_scales, uint8_t *out, int threads)
{
    if (!stream || !out)
        return LFM_EINVAL;
    job j = {full_scales ? 2 : 0, stream_seed(seed, stream), 0, 0, d_sigma, 0.f, out};
    run_parallel(j, nblocks, threads);
    return LFM_OK;
}

int lfm_synth_q6k_blocks(uint64_t seed, const char *stream, uint64_t nblocks, float d_sigma,
                         uint8_t *out, int threads)
{
    return lfm_synth_q6k_blocks_ex(seed, stream, nblocks, d_sigma, 0, out, threads);
}

int lfm_synth_normal_f32(uint64_t seed, const char *stream, uint64_t n, float mean, float sigma,
                         float *out, int threads)
{
    if (!stream || !out)
        return LFM_EINVAL;
    const uint64_t pairs = n / 2;
    job j = {1, stream_seed(seed, stream), 0, 0, mean, sigma, out};
    run_parallel(j, pairs, threads);
    if (n & 1) { /* odd tail: first value of the next pair */
        uint64_t s = j.tseed + (pairs + 1) * 0xD1B54A32D192ED03ull;
        double z0, z1;
        normal_pair(&s, &z0, &z1);
        out[n - 1] = (float)(mean + sigma * z0);
    }
    return LFM_OK;
}

/* ---------------------------------------------------------------- model */
void lfm_synth_default_opts(lfm_synth_opts *o)
{
    o->seed = 0x9E3779B97F4A7C15ull;
    o->d_sigma = 1e-3f;
    o->norm_sigma = 0.02f;
    o->router_sigma = 0.02f;
    o->bias_sigma = 0.0f;
    o->conv_sigma = 0.1f;
    o->full_scales = 0;
}

static int layer_tensor_count(const lfm_hparams *hp, uint32_t l)
{
    int n = 2; /* attn_norm, ffn_norm */
    n += hp->kv_heads[l] > 0 ? 6 : 3;
    n += l < hp->dense_lead ? 3 : 5;
    return n;
}

int lfm_model_tensor_count(const lfm_hparams *hp)
{
    if (!hp || hp->n_layers > LFM_MAX_LAYERS)
        return -1;
    int n = 2;
    for (uint32_t l = 0; l < hp->n_layers; ++l)
        n += layer_tensor_count(hp, l);
    return n;
}

static void set_desc(lfm_tensor_desc *d, const char *name, uint32_t type, uint32_t nd,
                     uint64_t n0, uint64_t n1, uint64_t n2, uint32_t kind, float sigma)
{
    memset(d, 0, sizeof(*d));
    snprintf(d->name, sizeof(d->name), "%s", name);
    d->ggml_type = type;
    d->n_dims = nd;
    d->ne[0] = n0;
    d->ne[1] = nd > 1 ? n1 : 1;
    d->ne[2] = nd > 2 ? n2 : 1;
    d->ne[3] = 1;
    d->kind = kind;
    d->sigma = sigma;
}

int lfm_model_tensor_desc(const lfm_hparams *hp, const lfm_synth_opts *o, int index,
                          lfm_tensor_desc *out)
{
    lfm_synth_opts def;
    if (!o) {
        lfm_synth_default_opts(&def);
        o = &def;
    }
    if (!hp || !out || index < 0)
        return LFM_EINVAL;
    const uint64_t dim = hp->dim, V = hp->vocab, hdkv_unit = hp->head_dim;
    const uint32_t Q6 = LFM_GGML_TYPE_Q6_K, F32 = LFM_GGML_TYPE_F32;
    if (index == 0) {
        set_desc(out, "token_embd.weight", Q6, 2, dim, V, 0, 0, 0.f);
        return LFM_OK;
    }
    if (index == 1) {
        set_desc(out, "token_embd_norm.weight", F32, 1, dim, 0, 0, 1, o->norm_sigma);
        return LFM_OK;
    }
    int i = index - 2;
    for (uint32_t l = 0; l < hp->n_layers; ++l) {
        const int cnt = layer_tensor_count(hp, l);
        if (i >= cnt) {
            i -= cnt;
            continue;
        }
        char nm[96];
#define NM(s) (snprintf(nm, sizeof(nm), "blk.%u." s, (unsigned)l), nm)
        const uint64_t hdkv = hdkv_unit * hp->kv_heads[l];
        if (i == 0) {
            set_desc(out, NM("attn_norm.weight"), F32, 1, dim, 0, 0, 1, o->norm_sigma);
            return LFM_OK;
        }
        if (i == 1) {
            set_desc(out, NM("ffn_norm.weight"), F32, 1, dim, 0, 0, 1, o->norm_sigma);
            return LFM_OK;
        }
        i -= 2;
        if (hp->kv_heads[l] > 0) {
            switch (i) {
            case 0: set_desc(out, NM("attn_q.weight"), Q6, 2, dim, dim, 0, 0, 0.f); return LFM_OK;
            case 1: set_desc(out, NM("attn_k.weight"), Q6, 2, dim, hdkv, 0, 0, 0.f); return LFM_OK;
            case 2: set_desc(out, NM("attn_v.weight"), Q6, 2, dim, hdkv, 0, 0, 0.f); return LFM_OK;
            case 3: set_desc(out, NM("attn_output.weight"), Q6, 2, dim, dim, 0, 0, 0.f); return LFM_OK;
            case 4:
                set_desc(out, NM("attn_q_norm.weight"), F32, 1, hp->head_dim, 0, 0, 1, o->norm_sigma);
                return LFM_OK;
            case 5:
                set_desc(out, NM("attn_k_norm.weight"), F32, 1, hp->head_dim, 0, 0, 1, o->norm_sigma);
                return LFM_OK;
            }
            i -= 6;
        } else {
            switch (i) {
            case 0:
                set_desc(out, NM("shortconv.in_proj.weight"), Q6, 2, dim, 3 * dim, 0, 0, 0.f);
                return LFM_OK;
            case 1:
                set_desc(out, NM("shortconv.out_proj.weight"), Q6, 2, dim, dim, 0, 0, 0.f);
                return LFM_OK;
            case 2:
                set_desc(out, NM("shortconv.conv.weight"), F32, 2, hp->conv_l_cache, dim, 0, 2,
                         o->conv_sigma);
                return LFM_OK;
            }
            i -= 3;
        }
        if (l < hp->dense_lead) {
            switch (i) {
            case 0: set_desc(out, NM("ffn_gate.weight"), Q6, 2, dim, hp->n_ff, 0, 0, 0.f); return LFM_OK;
            case 1: set_desc(out, NM("ffn_up.weight"), Q6, 2, dim, hp->n_ff, 0, 0, 0.f); return LFM_OK;
            case 2: set_desc(out, NM("ffn_down.weight"), Q6, 2, hp->n_ff, dim, 0, 0, 0.f); return LFM_OK;
            }
        } else {
            switch (i) {
            case 0:
                set_desc(out, NM("ffn_gate_inp.weight"), F32, 2, dim, hp->n_expert, 0, 2,
                         o->router_sigma);
                return LFM_OK;
            case 1:
                set_desc(out, NM("exp_probs_b.bias"), F32, 1, hp->n_expert, 0, 0,
                         o->bias_sigma > 0.f ? 2 : 3, o->bias_sigma);
                return LFM_OK;
            case 2:
                set_desc(out, NM("ffn_gate_exps.weight"), Q6, 3, dim, hp->expert_ff, hp->n_expert, 0, 0.f);
                return LFM_OK;
            case 3:
                set_desc(out, NM("ffn_up_exps.weight"), Q6, 3, dim, hp->expert_ff, hp->n_expert, 0, 0.f);
                return LFM_OK;
            case 4:
                set_desc(out, NM("ffn_down_exps.weight"), Q6, 3, hp->expert_ff, dim, hp->n_expert, 0, 0.f);
                return LFM_OK;
            }
        }
#undef NM
        return LFM_EINTERNAL;
    }
    return LFM_ERANGE;
}

size_t lfm_tensor_nbytes(const lfm_tensor_desc *d)
{
    if (!d)
        return 0;
    uint64_t n = 1;
    for (uint32_t i = 0; i < d->n_dims && i < 4; ++i)
        n *= d->ne[i];
    if (d->ggml_type == LFM_GGML_TYPE_Q6_K)
        return (size_t)(n / 256 * 210);
    return (size_t)(n * 4);
}

int lfm_synth_tensor(const lfm_synth_opts *o, const lfm_tensor_desc *d, void *out, size_t cap,
                     int threads)
{
    lfm_synth_opts def;
    if (!o) {
        lfm_synth_default_opts(&def);
        o = &def;
    }
    if (!d || !out)
        return LFM_EINVAL;
    const size_t nbytes = lfm_tensor_nbytes(d);
    if (cap < nbytes)
        return LFM_ERANGE;
    if (d->ggml_type == LFM_GGML_TYPE_Q6_K) {
        if (d->ne[0] % 256)
            return LFM_EINVAL;
        return lfm_synth_q6k_blocks_ex(o->seed, d->name, nbytes / 210, o->d_sigma, (int)o->full_scales,
                                       (uint8_t *)out, threads);
    }
    const uint64_t n = nbytes / 4;
    switch (d->kind) {
    case 1: return lfm_synth_normal_f32(o->seed, d->name, n, 1.0f, d->sigma, (float *)out, threads);
    case 2: return lfm_synth_normal_f32(o->seed, d->name, n, 0.0f, d->sigma, (float *)out, threads);
    case 3: memset(out, 0, nbytes); return LFM_OK;
    default: return LFM_EINVAL;
    }
}
