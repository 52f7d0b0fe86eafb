// lfm_prefill.hip -- gfx950 MFMA kernels of the multi-token (prefill) path.
//
// Prefill is the one place the LFM2 token loop is a dense contraction: every
// projection multiplies a Q6_K weight by T activation columns.  The GEMM here
// runs on the matrix cores (v_mfma_f32_32x32x16_f16):
//   * the weight tile is decoded in LDS to binary16 values sc * (q - 32), which
//     are exact whenever |sc * (q - 32)| <= 2048 (and within 1/2 ulp otherwise);
//   * the super-block scale d multiplies each 256-wide block's partial product
//     in fp32 (one FMA per accumulator per block);
//   * activations are split into binary16 hi + lo (x = hi + lo to ~22 bits), and
//     both halves go through the matrix cores, so results are close to an fp32
//     matvec (the reference's prefill is its f32 q6k_prompt path,
//     engine/src/kernels.rs:1039-1044 over ops.rs:350-373).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kargs.h"
#include "q6_device.h"
#include "wave_ops.h"

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

#define WG_THREADS 256
#define GM 128         // weight rows per workgroup
#define GN 128         // token columns per workgroup
#define GK 128         // K elements per LDS stage (half a Q6_K block)
#define LDS_ROW 136    // halves per LDS row (GK + 8: 272 B rows keep 16-B reads conflict-free)


// Split an f32 into binary16 hi + lo with hi = fp16(x), lo = fp16(x - hi).
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// RMSNorm (optional) of T rows of x [T][K], then a binary16 hi/lo split of
// x / scale with scale = 2^(e - 14) for max|x| = m * 2^e (so |x / scale| < 2^14).
// One workgroup per token row.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_split_rows(const SplitArgs a)
{
    const uint32_t t = blockIdx.x;
    if (t >= a.T)
        return;
    const float *x = a.x + (size_t)t * a.K;
    __shared__ float red[4], redm[4];
    float ss = 0.f;
    for (uint32_t k = threadIdx.x; k < a.K; k += WG_THREADS)
        ss += x[k] * x[k];
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float inv = a.norm_w ? 1.0f / sqrtf(tot / (float)a.K + a.eps) : 1.0f;
    float amax = 0.f;
    for (uint32_t k = threadIdx.x; k < a.K; k += WG_THREADS) {
        const float v = a.norm_w ? x[k] * inv * a.norm_w[k] : x[k];
        amax = fmaxf(amax, fabsf(v));
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0)
        redm[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    int e = 0;
    if (amax > 0.f && amax <= 3.0e38f)
        frexpf(amax, &e);
    const float scale = amax > 0.f ? ldexpf(1.0f, e - 14) : 1.0f, rs = 1.0f / scale;
    if (threadIdx.x == 0)
        a.scale[t] = scale;
    _Float16 *hi = reinterpret_cast<_Float16 *>(a.hi) + (size_t)t * a.K;
    _Float16 *lo = reinterpret_cast<_Float16 *>(a.lo) + (size_t)t * a.K;
    for (uint32_t k = threadIdx.x; k < a.K; k += WG_THREADS) {
        const float v = (a.norm_w ? x[k] * inv * a.norm_w[k] : x[k]) * rs;
        split_f16(v, hi[k], lo[k]);
    }
}

// Decode one lane chunk (32 weights of block b, chunk c) into binary16 values
// sc * (q - 32) at LDS row `dst` (positions s*32 + l0 + i within the half block).
__device__ __forceinline__ void chunk_to_lds(const Q6T &t, uint32_t row, uint32_t b, uint32_t c,
                                             _Float16 *dst)
{
    const size_t nblk = (size_t)t.rows * t.nb;
    const size_t blk = (size_t)row * t.nb + b;
    const uint4 ql = *reinterpret_cast<const uint4 *>(t.base + blk * 128 + c * 16);
    const uint2 qh = *reinterpret_cast<const uint2 *>(t.base + nblk * 128 + blk * 64 + c * 8);
    const uint32_t sc = *reinterpret_cast<const uint32_t *>(t.base + nblk * 192 + blk * 16 + (c >> 1) * 4);
    const uint32_t l0 = (c & 3) * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int scv = (int)(int8_t)(sc >> (8 * s));
        half8 v;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t A = j ? ql.y : ql.x, B = j ? ql.w : ql.z, H = j ? qh.y : qh.x;
            uint32_t q;
            switch (s) {
            case 0: q = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u); break;
            case 1: q = (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u); break;
            case 2: q = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u); break;
            default: q = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u); break;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
                v[j * 4 + i] = (_Float16)(float)(scv * ((int)((q >> (8 * i)) & 0xFFu) - 32));
        }
        *reinterpret_cast<half8 *>(dst + s * 32 + l0) = v;
    }
}

// C[n][row] (+)= sum_k W[row][k] * X[n][k] for weight rows [0, w.rows) and token
// columns n < ntok.  Column n reads activation row (tok ? tok[n] : n) and writes
// output row (slot ? slot[n] : n).  Tiles of 128 rows x 128 tokens per
// workgroup; each wave owns 64 x 64 (2 x 2 MFMA 32x32 tiles).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_gemm_q6(const GemmArgs a)
{
    const uint32_t z = blockIdx.z;
    const uint32_t m0 = blockIdx.x * GM, n0 = blockIdx.y * GN;
    const uint32_t ntok = a.counts ? a.counts[z] : a.ntok;
    if (m0 >= a.zrows || n0 >= ntok)
        return;
    const uint32_t rbase = z * a.zrows;
    const uint32_t *tokl = a.tok ? a.tok + (size_t)z * a.list_stride : nullptr;
    const uint32_t *slotl = a.slot ? a.slot + (size_t)z * a.list_stride : nullptr;
    const _Float16 *xh = reinterpret_cast<const _Float16 *>(a.x_hi);
    const _Float16 *xl = reinterpret_cast<const _Float16 *>(a.x_lo);
    __shared__ __attribute__((aligned(16))) _Float16 As[GM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) _Float16 Bh[GN * LDS_ROW];
    __shared__ __attribute__((aligned(16))) _Float16 Bl[GN * LDS_ROW];
    __shared__ float dsh[GM];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t wm = (wave & 1) * 64, wn = (wave >> 1) * 64;
    const uint32_t K = a.w.nb * 256;
    floatx16 acc[2][2], tmp[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.f, tmp[i][j][e] = 0.f;

    for (uint32_t kb = 0; kb < a.w.nb; ++kb) {
        for (uint32_t h = 0; h < 2; ++h) {
            // A: 128 rows x 4 chunks of this half block, 2 (row, chunk) units per thread
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint32_t unit = tid + u * WG_THREADS, r = unit >> 2, c = h * 4 + (unit & 3);
                const uint32_t row = rbase + (m0 + r < a.zrows ? m0 + r : a.zrows - 1);
                chunk_to_lds(a.w, row, kb, c, As + r * LDS_ROW);
                if (h == 0 && (unit & 3) == 0) {
                    const size_t nblk = (size_t)a.w.rows * a.w.nb;
                    dsh[r] = half_bits_to_float(
                        reinterpret_cast<const uint16_t *>(a.w.base + nblk * 208)[(size_t)row * a.w.nb + kb]);
                }
            }
            // B: 128 tokens x 128 k of hi and lo (16 B per piece, 8 + 8 pieces per thread)
            const uint32_t k0 = kb * 256 + h * 128;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t piece = tid + u * WG_THREADS, n = piece >> 4, kk = (piece & 15) * 8;
                const uint32_t col = n0 + n < ntok ? n0 + n : ntok - 1;
                const uint32_t src = tokl ? tokl[col] : col;
                *reinterpret_cast<uint4 *>(Bh + n * LDS_ROW + kk) =
                    *reinterpret_cast<const uint4 *>(xh + (size_t)src * K + k0 + kk);
                *reinterpret_cast<uint4 *>(Bl + n * LDS_ROW + kk) =
                    *reinterpret_cast<const uint4 *>(xl + (size_t)src * K + k0 + kk);
            }
            __syncthreads();
#pragma unroll
            for (int ks = 0; ks < GK / 16; ++ks) {
                const uint32_t ko = ks * 16 + (lane >> 5) * 8;
                half8 af[2], bh[2], bl[2];
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    af[i] = *reinterpret_cast<const half8 *>(As + (wm + i * 32 + (lane & 31)) * LDS_ROW + ko);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    bh[j] = *reinterpret_cast<const half8 *>(Bh + (wn + j * 32 + (lane & 31)) * LDS_ROW + ko);
                    bl[j] = *reinterpret_cast<const half8 *>(Bl + (wn + j * 32 + (lane & 31)) * LDS_ROW + ko);
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bh[j], tmp[i][j], 0, 0, 0);
                        tmp[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bl[j], tmp[i][j], 0, 0, 0);
                    }
            }
            if (h == 1) {
                // end of the super-block: acc += d[row] * partial
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const uint32_t r = wm + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                        const float dv = dsh[r];
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            acc[i][j][e] += dv * tmp[i][j][e];
                            tmp[i][j][e] = 0.f;
                        }
                    }
            }
            __syncthreads();
        }
    }
    // epilogue: lane holds rows 8*(e/4) + 4*(lane/32) + e%4 of column lane%32
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t n = n0 + wn + j * 32 + (lane & 31);
        if (n >= ntok)
            continue;
        const uint32_t orow = slotl ? slotl[n] : n;
        const float xs = a.xscale[tokl ? tokl[n] : n];
        float *out = a.c + (size_t)orow * a.ldc + a.col0;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t r = m0 + wm + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                const float v = acc[i][j][e] * xs;
                if (r < a.zrows)
                    out[r] = a.mode ? out[r] + v : v;
            }
    }
}

// ------------------------------------------------------------------ short conv
// The LFM2 short conv keeps only the previous two values of bx = B*X, so each
// (t, ch) output depends on inputs t-2, t-1, t only: the T tokens of a chunk are
// computed in parallel with the reference's per-element operation order
// (lfm.rs:464-533: co = ((0 + s0*w0) + s1*w1) + bx*w2, y = C*co, no contraction).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_conv_prefill(const ConvPrefillArgs a)
{
#pragma clang fp contract(off)
    const uint32_t ch = blockIdx.x * WG_THREADS + threadIdx.x;
    const uint32_t t = blockIdx.y;
    if (ch >= a.dim || t >= a.T)
        return;
    const uint32_t D3 = 3 * a.dim;
    auto bx_at = [&](int tt) -> float {
        if (tt >= 0)
            return a.bcx[(size_t)tt * D3 + ch] * a.bcx[(size_t)tt * D3 + 2 * a.dim + ch];
        return a.state[ch * 2 + (tt == -2 ? 0 : 1)];
    };
    const float s0 = bx_at((int)t - 2), s1 = bx_at((int)t - 1), bx = bx_at((int)t);
    const float *w3 = a.conv_w + ch * 3;
    float co = 0.0f;
    co = co + s0 * w3[0];
    co = co + s1 * w3[1];
    co = co + bx * w3[2];
    a.y[(size_t)t * a.dim + ch] = a.bcx[(size_t)t * D3 + a.dim + ch] * co;
}

// New conv state after the chunk: (bx[T-2], bx[T-1]) (or (s1, bx[0]) for T = 1).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_conv_state(const ConvPrefillArgs a)
{
#pragma clang fp contract(off)
    const uint32_t ch = blockIdx.x * WG_THREADS + threadIdx.x;
    if (ch >= a.dim)
        return;
    const uint32_t D3 = 3 * a.dim;
    const float last = a.bcx[(size_t)(a.T - 1) * D3 + ch] * a.bcx[(size_t)(a.T - 1) * D3 + 2 * a.dim + ch];
    const float prev = a.T >= 2 ? a.bcx[(size_t)(a.T - 2) * D3 + ch] * a.bcx[(size_t)(a.T - 2) * D3 + 2 * a.dim + ch]
                                : a.state[ch * 2 + 1];
    a.state[ch * 2] = prev;
    a.state[ch * 2 + 1] = last;
}

// ------------------------------------------------------------------ attention

// Per token: q heads and k heads RMS-normed over head_dim and NEOX-rotated at
// position start + t (table row), q written back, K and V rounded to binary16 and
// stored in the cache (lfm.rs:360-393).  One wave per head.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_rope_kv_prefill(const RopeKvArgs a)
{
    const uint32_t t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (t >= a.T)
        return;
    const uint32_t dim = a.heads * 64, hdkv = a.kv * 64, pos = a.start + t;
    float *row = a.qkv + (size_t)t * (dim + 2 * hdkv);
    const float *cs = a.rope + (size_t)pos * 64;
    for (uint32_t h = wave; h < a.heads + a.kv; h += 4) {
        const bool isq = h < a.heads;
        float v = row[(isq ? 0 : dim) + (isq ? h : h - a.heads) * 64 + lane];
        const float ss = wave_sum(v * v);
        const float inv = 1.0f / sqrtf(ss / 64.0f + a.eps);
        v *= inv * (isq ? a.q_norm : a.k_norm)[lane];
        const float other = __shfl_xor(v, 32, 64);
        const uint32_t p = lane & 31;
        const float c = cs[2 * p], s = cs[2 * p + 1];
        const float r = lane < 32 ? v * c - other * s : other * s + v * c;
        if (isq) {
            row[h * 64 + lane] = r;
        } else {
            const uint32_t kh = h - a.heads;
            const size_t off = ((size_t)kh * a.ctx + pos) * 64 + lane;
            a.kcache[off] = __builtin_bit_cast(uint16_t, (_Float16)r);
            a.vcache[off] = __builtin_bit_cast(uint16_t, (_Float16)row[dim + hdkv + kh * 64 + lane]);
        }
    }
}

// Causal attention (lfm.rs:395-437): a workgroup takes 64 queries of one kv head;
// thread = (query, q head of the group).  Keys/values stream through LDS in
// blocks of 64 positions; online softmax in fp32.
#define PQ 64
#define PK 64
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_attn_prefill(const AttnPrefillArgs a)
{
    const uint32_t kh = blockIdx.y, q0 = blockIdx.x * PQ;
    if (q0 >= a.T)
        return;
    const uint32_t G = a.heads / a.kv, dim = a.heads * 64, hdkv = a.kv * 64;
    const uint32_t tid = threadIdx.x, qi = tid & (PQ - 1), g = tid >> 6;
    __shared__ __attribute__((aligned(16))) float Ks[PK][64];
    __shared__ __attribute__((aligned(16))) float Vs[PK][64];
    const uint32_t t = q0 + qi;
    const bool live = t < a.T && g < G;
    const uint32_t pos = a.start + (t < a.T ? t : a.T - 1);
    float q[64], acc[64];
    const float *qrow = a.qkv + (size_t)(t < a.T ? t : a.T - 1) * (dim + 2 * hdkv) + (kh * G + (g < G ? g : 0)) * 64;
#pragma unroll
    for (int d = 0; d < 64; ++d) {
        q[d] = qrow[d] * a.scale;
        acc[d] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    const uint32_t last_pos = a.start + min(q0 + PQ, a.T) - 1; // highest position in this block
    for (uint32_t k0 = 0; k0 <= last_pos; k0 += PK) {
        __syncthreads();
        for (uint32_t u = tid; u < PK * 64; u += WG_THREADS) {
            const uint32_t kk = u >> 6, d = u & 63;
            const uint32_t kp = k0 + kk <= last_pos ? k0 + kk : last_pos;
            const size_t off = ((size_t)kh * a.ctx + kp) * 64 + d;
            Ks[kk][d] = (float)__builtin_bit_cast(_Float16, a.kcache[off]);
            Vs[kk][d] = (float)__builtin_bit_cast(_Float16, a.vcache[off]);
        }
        __syncthreads();
        if (!live)
            continue;
        const uint32_t nk = min((uint32_t)PK, pos + 1 > k0 ? pos + 1 - k0 : 0u);
        for (uint32_t kk = 0; kk < nk; ++kk) {
            float s = 0.f;
#pragma unroll
            for (int d = 0; d < 64; ++d)
                s += q[d] * Ks[kk][d];
            if (s > m) {
                const float r = expf(m - s);
                l *= r;
#pragma unroll
                for (int d = 0; d < 64; ++d)
                    acc[d] *= r;
                m = s;
            }
            const float p = expf(s - m);
            l += p;
#pragma unroll
            for (int d = 0; d < 64; ++d)
                acc[d] += p * Vs[kk][d];
        }
    }
    if (!live)
        return;
    float *o = a.out + (size_t)t * dim + (kh * G + g) * 64;
    const float rl = 1.0f / l;
#pragma unroll
    for (int d = 0; d < 64; ++d)
        o[d] = acc[d] * rl;
}

// ------------------------------------------------------------------ FFN pieces
// sw = g / (1 + exp(-g)) * u (lfm.rs:578-582), then the binary16 hi/lo split for
// the down projection with a per-row power-of-two scale.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_swiglu_split(const SwigluSplitArgs a)
{
    const uint32_t t = blockIdx.x;
    if (t >= a.T)
        return;
    const float *g = a.g + (size_t)t * a.ff, *u = a.u + (size_t)t * a.ff;
    __shared__ float redm[4];
    float amax = 0.f;
    for (uint32_t k = threadIdx.x; k < a.ff; k += WG_THREADS) {
        const float gv = g[k];
        amax = fmaxf(amax, fabsf(gv / (1.0f + expf(-gv)) * u[k]));
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0)
        redm[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    int e = 0;
    if (amax > 0.f && amax <= 3.0e38f)
        frexpf(amax, &e);
    const float scale = amax > 0.f ? ldexpf(1.0f, e - 14) : 1.0f, rs = 1.0f / scale;
    if (threadIdx.x == 0)
        a.scale[t] = scale;
    _Float16 *hi = reinterpret_cast<_Float16 *>(a.hi) + (size_t)t * a.ff;
    _Float16 *lo = reinterpret_cast<_Float16 *>(a.lo) + (size_t)t * a.ff;
    for (uint32_t k = threadIdx.x; k < a.ff; k += WG_THREADS) {
        const float gv = g[k];
        split_f16(gv / (1.0f + expf(-gv)) * u[k] * rs, hi[k], lo[k]);
    }
}

// Router logits for T tokens (lfm.rs:599-607): a workgroup takes 16 tokens.
// Each wave first finds the RMSNorm scale of 4 of them; then 256-wide slices of
// x . w and of the f32 router rows are staged in LDS and thread (token, e)
// accumulates its dot products in k order; logits = inv * sum.
#define RT_TOK 16
#define RT_K 256
#define RT_EMAX 64
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_router_prefill(const RouterPrefillArgs a)
{
    __shared__ float inv[RT_TOK];
    __shared__ float xs[RT_TOK][RT_K + 1];
    __shared__ float ws[RT_EMAX][RT_K + 1];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t t0 = blockIdx.x * RT_TOK;
    for (uint32_t j = 0; j < RT_TOK / 4; ++j) {
        const uint32_t tt = wave * (RT_TOK / 4) + j, t = t0 + tt;
        if (t < a.T) { // uniform across the wave
            const float *x = a.x + (size_t)t * a.dim;
            float ss = 0.f;
            for (uint32_t k = lane; k < a.dim; k += 64)
                ss += x[k] * x[k];
            ss = wave_sum(ss);
            if (lane == 0)
                inv[tt] = 1.0f / sqrtf(ss / (float)a.dim + a.eps);
        }
    }
    const uint32_t tt = tid / 16, eg = tid % 16;
    float acc[RT_EMAX / 16];
#pragma unroll
    for (int j = 0; j < RT_EMAX / 16; ++j)
        acc[j] = 0.f;
    for (uint32_t k0 = 0; k0 < a.dim; k0 += RT_K) {
        __syncthreads();
        for (uint32_t u = tid; u < RT_TOK * RT_K; u += WG_THREADS) {
            const uint32_t r = u / RT_K, kk = u % RT_K, t = t0 + r;
            xs[r][kk] = t < a.T ? a.x[(size_t)t * a.dim + k0 + kk] * a.norm_w[k0 + kk] : 0.f;
        }
        for (uint32_t u = tid; u < a.n_expert * RT_K; u += WG_THREADS) {
            const uint32_t e = u / RT_K, kk = u % RT_K;
            ws[e][kk] = a.w[(size_t)e * a.dim + k0 + kk];
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < RT_EMAX / 16; ++j) {
            const uint32_t e = eg + 16 * j;
            if (e < a.n_expert) {
                float s = acc[j];
                for (uint32_t kk = 0; kk < RT_K; ++kk)
                    s += xs[tt][kk] * ws[e][kk];
                acc[j] = s;
            }
        }
    }
    const uint32_t t = t0 + tt;
    if (t < a.T)
#pragma unroll
        for (int j = 0; j < RT_EMAX / 16; ++j) {
            const uint32_t e = eg + 16 * j;
            if (e < a.n_expert)
                a.logits[(size_t)t * a.n_expert + e] = inv[tt] * acc[j];
        }
}

// Top-k per token (the decode routing rule, wave_route): one wave per token
// stores the selected ids and weights [t][4] (unused ranks: id 0, weight 0).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_route_topk(const RouteGroupArgs a)
{
    const uint32_t lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) // uniform across the wave
        return;
    Route r;
    r.logits = a.logits + (size_t)t * a.n_expert;
    r.bias = a.bias;
    r.n_expert = a.n_expert;
    r.n_used = a.n_used;
    r.sel_out = nullptr;
    const Routed rt = wave_route(r);
    if (lane < 4) {
        a.sel[(size_t)t * 4 + lane] = rt.id(lane);
        a.wsel[(size_t)t * 4 + lane] = lane < a.n_used ? rt.w(lane) : 0.f;
    }
}

// Per expert (one workgroup each) the (token, rank) pairs that selected it, in
// token order: tok[e][i] = token, slot[e][i] = token * 4 + rank; counts[e].
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_route_group(const RouteGroupArgs a)
{
    const uint32_t e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ uint32_t wave_cnt[4];
    __shared__ uint32_t base;
    if (tid == 0)
        base = 0;
    __syncthreads();
    for (uint32_t t0 = 0; t0 < a.T; t0 += WG_THREADS) {
        const uint32_t t = t0 + tid;
        uint32_t rank_of_e = 4; // 4: not selected
        if (t < a.T) {
            const uint4 s4 = *reinterpret_cast<const uint4 *>(a.sel + (size_t)t * 4);
            const uint32_t ids[4] = {s4.x, s4.y, s4.z, s4.w};
            for (int r = (int)a.n_used - 1; r >= 0; --r)
                if (ids[r] == e)
                    rank_of_e = (uint32_t)r;
        }
        const bool hit = rank_of_e < 4;
        const uint64_t mask = __ballot(hit);
        const uint32_t before = __popcll(mask & ((1ull << lane) - 1ull));
        if (lane == 0)
            wave_cnt[wave] = __popcll(mask);
        __syncthreads();
        uint32_t off = base;
        for (uint32_t w = 0; w < wave; ++w)
            off += wave_cnt[w];
        if (hit) {
            a.tok[(size_t)e * a.list_stride + off + before] = t;
            a.slot[(size_t)e * a.list_stride + off + before] = t * 4 + rank_of_e;
        }
        __syncthreads();
        if (tid == 0)
            base += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
        __syncthreads();
    }
    if (tid == 0)
        a.counts[e] = base;
}

// x[t][k] += ((((0 + D[t,0][k] w0) + D[t,1][k] w1) + ...) in rank order
// (lfm.rs:645-668, no contraction).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_combine_prefill(const CombinePrefillArgs a)
{
#pragma clang fp contract(off)
    const uint32_t k = blockIdx.x * WG_THREADS + threadIdx.x, t = blockIdx.y;
    if (k >= a.dim || t >= a.T)
        return;
    float s = 0.0f;
    for (uint32_t r = 0; r < a.n_used; ++r)
        s = s + a.d[((size_t)t * 4 + r) * a.dim + k] * a.wsel[(size_t)t * 4 + r];
    float *x = a.x + (size_t)t * a.dim + k;
    *x = *x + s;
}

// Token embeddings of T ids (lfm.rs:310-320): row ids[t] of the Q6_K table,
// dequantized exactly; one wave per row (8 lanes per 256-wide block).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_embed_rows(const EmbedRowsArgs a)
{
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= a.T)
        return;
    const uint32_t tok = a.ids[t];
    for (uint32_t u = lane; u < a.emb.nb * 8; u += 64) {
        const uint32_t b = u >> 3, c = u & 7;
        float v[32];
        lane_dequant(load_lane(a.emb, tok, b, c), v);
        float *o = a.x + (size_t)t * a.emb.nb * 256;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                o[lane_pos(b, c, s, i)] = v[s * 8 + i];
    }
}
