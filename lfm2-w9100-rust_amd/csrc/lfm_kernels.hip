// lfm_kernels.hip -- hand-written gfx950 (CDNA4, wave64) kernels of the LFM2
// Q6_K decode step.  Compiled to a code object (hipcc --genco) and launched by
// engine.cpp with hipModuleLaunchKernel; one decode step is captured into a
// hipGraph.  Every kernel reads the token/position from the device-resident
// DevState, so a captured step replays at any position.
//
// Reference semantics (Amidwestnoob/lfm2-w9100-rust):
//   Q6_K element decode           engine/src/q6k.rs:74-146, kernels.rs:765-794
//   matvec                        engine/src/q6k.rs:167-183, kernels.rs:832-1025
//   RMSNorm                       engine/src/lfm.rs:231-244, kernels.rs:576-634
//   per-head norm + NEOX RoPE     engine/src/lfm.rs:248-286, kernels.rs:636-670
//   KV f16 RNE write              engine/src/lfm.rs:375-393, kernels/resident.rs:119-169
//   decode attention              engine/src/lfm.rs:395-437, kernels.rs:672-763
//   short conv                    engine/src/lfm.rs:450-533, kernels/resident.rs:33-56
//   router / top-k                engine/src/lfm.rs:599-637, kernels/resident.rs:58-99
//   SwiGLU                        engine/src/lfm.rs:578-582, kernels.rs:543-550
//   expert combine                engine/src/lfm.rs:645-668, kernels/resident.rs:101-117
//   embedding                     engine/src/lfm.rs:310-320, kernels/resident.rs:7-18
//   argmax                        engine/src/main.rs:112-141, kernels/persistent.rs:11-53
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kargs.h"

#define WG_THREADS 256
#define ATT_CH 128  // attention positions per workgroup
#define ATT_KROW 72 // LDS row stride of a K row, in halves (144 B: conflict-free 16-B reads)

// ---------------------------------------------------------------- wave helpers
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o < v ? o : v;
    }
    return v;
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint16_t float_to_half_bits(float f)
{
    // v_cvt_f16_f32: IEEE round-to-nearest-even with gradual underflow.
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// ------------------------------------------------------------- Q6_K lane data
// A wave reads a row as 8 lanes per super-block: lane c of block b owns the 32
// weights at  b*256 + h*128 + s*32 + l0 + i  (h = c/4, l0 = (c%4)*8, s, i < 8).
struct Lane {
    uint4 ql;    // ql[h*64+l0 .. +8] ++ ql[h*64+32+l0 .. +8]
    uint2 qh;    // qh[h*32+l0 .. +8]
    uint32_t sc; // scales of sub-rows s = 0..3 for this (h, l0/16)
    uint32_t d;  // binary16 super-block scale
};

__device__ __forceinline__ Lane load_lane(const Q6T &t, uint32_t row, uint32_t b, uint32_t c)
{
    const size_t nblk = (size_t)t.rows * t.nb;
    const size_t blk = (size_t)row * t.nb + b;
    Lane w;
    w.ql = *reinterpret_cast<const uint4 *>(t.base + blk * 128 + c * 16);
    w.qh = *reinterpret_cast<const uint2 *>(t.base + nblk * 128 + blk * 64 + c * 8);
    w.sc = *reinterpret_cast<const uint32_t *>(t.base + nblk * 192 + blk * 16 + (c >> 1) * 4);
    w.d = reinterpret_cast<const uint16_t *>(t.base + nblk * 208)[blk];
    return w;
}

// 6-bit codes of sub-row s as four bytes per word (j = 0: i 0..3, j = 1: i 4..7).
__device__ __forceinline__ uint32_t lane_codes(const Lane &w, int s, int j)
{
    const uint32_t A = j ? w.ql.y : w.ql.x;
    const uint32_t B = j ? w.ql.w : w.ql.z;
    const uint32_t H = j ? w.qh.y : w.qh.x;
    switch (s) {
    case 0: return (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
    case 1: return (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
    case 2: return ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
    default: return ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
    }
}

// Activation values of a lane's 32 positions plus 32 * (sum of each group of 8).
struct LaneX {
    float v[32];
    float s32[4];
};

__device__ __forceinline__ void load_lanex(LaneX &X, const float *x, uint32_t b, uint32_t c)
{
    const uint32_t base = b * 256 + (c >> 2) * 128 + (c & 3) * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const float4 a = *reinterpret_cast<const float4 *>(x + base + s * 32);
        const float4 bb = *reinterpret_cast<const float4 *>(x + base + s * 32 + 4);
        X.v[s * 8 + 0] = a.x, X.v[s * 8 + 1] = a.y, X.v[s * 8 + 2] = a.z, X.v[s * 8 + 3] = a.w;
        X.v[s * 8 + 4] = bb.x, X.v[s * 8 + 5] = bb.y, X.v[s * 8 + 6] = bb.z, X.v[s * 8 + 7] = bb.w;
        float t = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            t += X.v[s * 8 + i];
        X.s32[s] = 32.f * t;
    }
}

__device__ __forceinline__ void zero_lanex(LaneX &X)
{
#pragma unroll
    for (int i = 0; i < 32; ++i)
        X.v[i] = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s)
        X.s32[s] = 0.f;
}

// Partial dot of one lane: d * sum_s sc_s * sum_i (q_i - 32) x_i, with the -32
// folded into the precomputed group sums (q_i in 0..63 converted by byte).
__device__ __forceinline__ float lane_dot(const Lane &w, const LaneX &X)
{
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t q = lane_codes(w, s, j);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc += (float)((q >> (8 * i)) & 0xFFu) * X.v[s * 8 + j * 4 + i];
        }
        const float scv = (float)(int8_t)(w.sc >> (8 * s));
        part += scv * (acc - X.s32[s]);
    }
    return half_bits_to_float(w.d) * part;
}

// Exact element values of a lane: (d * sc) * (q - 32), three float multiplies
// as in q6k.rs:141-144 (keeps the reference's signed zeros).
__device__ __forceinline__ void lane_dequant(const Lane &w, float *out32)
{
    const float d = half_bits_to_float(w.d);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const float ds = d * (float)(int8_t)(w.sc >> (8 * s));
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t q = lane_codes(w, s, j);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                out32[s * 8 + j * 4 + i] = ds * (float)((int)((q >> (8 * i)) & 0xFFu) - 32);
        }
    }
}

__device__ __forceinline__ uint32_t lane_pos(uint32_t b, uint32_t c, int s, int i)
{
    return b * 256 + (c >> 2) * 128 + s * 32 + (c & 3) * 8 + i;
}

// ------------------------------------------------------------ input staging
// Copies (or, for the first kernel of a step, dequantizes the embedding row of
// DevState::tok into) LDS and applies RMSNorm in place:
// x * (1 / sqrt(sum x^2 / n + eps)) * w  (lfm.rs:231-244).
// Every workgroup computes the same sum in the same order.
__device__ void stage_x(const XSrc &src, float *xs, uint32_t n, const DevState *st, float *red)
{
    const uint32_t tid = threadIdx.x;
    if (src.embed) {
        const uint32_t tok = st->tok;
        for (uint32_t u = tid; u < n / 32; u += WG_THREADS) {
            const uint32_t b = u >> 3, c = u & 7;
            float v[32];
            lane_dequant(load_lane(src.emb, tok, b, c), v);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    xs[lane_pos(b, c, s, i)] = v[s * 8 + i];
        }
        __syncthreads();
        if (blockIdx.x == 0 && blockIdx.y == 0 && src.x_out)
            for (uint32_t i = tid; i < n; i += WG_THREADS)
                src.x_out[i] = xs[i];
    } else {
        for (uint32_t i = tid * 4; i < n; i += WG_THREADS * 4)
            *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(src.x + i);
        __syncthreads();
    }
    if (src.norm_w) {
        float ss = 0.f;
        for (uint32_t i = tid; i < n; i += WG_THREADS)
            ss += xs[i] * xs[i];
        ss = wave_sum(ss);
        if ((tid & 63) == 0)
            red[tid >> 6] = ss;
        __syncthreads();
        const float tot = ((red[0] + red[1]) + red[2]) + red[3];
        const float inv = 1.0f / sqrtf(tot / (float)n + src.eps);
        __syncthreads();
        for (uint32_t i = tid; i < n; i += WG_THREADS)
            xs[i] = xs[i] * inv * src.norm_w[i];
        __syncthreads();
    }
}

// ------------------------------------------------------------------ kernels
// Generic Q6_K matvec: y = W x or y += W x, x optionally RMS-normed.  ksplit
// waves share a row (nbw blocks each, combined in LDS in wave order).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_q6_matvec(const MatvecArgs a)
{
    if (a.st && a.st->halt)
        return;
    extern __shared__ float smem[];
    float *xs = smem;
    float *red = smem + a.in_dim;
    stage_x(a.src, xs, a.in_dim, a.st, red);
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t ks = a.ksplit, rpi = 4 / ks;
    const uint32_t slot = wave / ks, kp = wave % ks;
    const uint32_t bslot = lane >> 3, c = lane & 7;
    const uint32_t b = kp * a.nbw + bslot;
    const bool active = bslot < a.nbw && b < a.w.nb;
    LaneX X;
    if (active)
        load_lanex(X, xs, b, c);
    else
        zero_lanex(X);
    const uint32_t rows = a.w.rows;
    const uint32_t ngroups = (rows + rpi - 1) / rpi;
    for (uint32_t g = blockIdx.x; g < ngroups; g += gridDim.x) {
        const uint32_t row = g * rpi + slot;
        float p = 0.f;
        if (active && row < rows)
            p = lane_dot(load_lane(a.w, row, b, c), X);
        p = wave_sum(p);
        if (ks == 1) {
            if (lane == 0 && row < rows)
                a.y[row] = a.mode ? a.y[row] + p : p;
        } else {
            if (lane == 0)
                red[8 + wave] = p;
            __syncthreads();
            if (kp == 0 && lane == 0 && row < rows) {
                float s = 0.f;
                for (uint32_t k = 0; k < ks; ++k)
                    s += red[8 + slot * ks + k];
                a.y[row] = a.mode ? a.y[row] + s : s;
            }
            __syncthreads();
        }
    }
}

// Short-conv block, decode (lfm.rs:450-533 for n = 1): one wave per channel
// computes the in_proj rows B[ch], C[ch], X[ch], then
//   bx = B*X; co = ((0 + s0*w0) + s1*w1) + bx*w2; y = C*co; state = (s1, bx)
// in the reference's operation order with no contraction.
__device__ __forceinline__ void conv_step(float B, float C, float Xv, const float *w3, float *s2,
                                          float *y)
{
#pragma clang fp contract(off)
    const float bx = B * Xv;
    const float s0 = s2[0], s1 = s2[1];
    float co = 0.0f;
    co = co + s0 * w3[0];
    co = co + s1 * w3[1];
    co = co + bx * w3[2];
    *y = C * co;
    s2[0] = s1;
    s2[1] = bx;
}

extern "C" __global__ __launch_bounds__(WG_THREADS) void k_conv_inproj(const ConvInprojArgs a)
{
    if (a.st->halt)
        return;
    extern __shared__ float smem[];
    float *xs = smem;
    float *red = smem + a.dim;
    stage_x(a.src, xs, a.dim, a.st, red);
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.w.nb;
    LaneX X;
    if (active)
        load_lanex(X, xs, b, c);
    else
        zero_lanex(X);
    const uint32_t dim = a.dim;
    for (uint32_t ch = blockIdx.x * 4 + wave; ch < dim; ch += gridDim.x * 4) {
        float pb = 0.f, pc = 0.f, px = 0.f;
        if (active) {
            const Lane wb = load_lane(a.w, ch, b, c);
            const Lane wc = load_lane(a.w, dim + ch, b, c);
            const Lane wx = load_lane(a.w, 2 * dim + ch, b, c);
            pb = lane_dot(wb, X);
            pc = lane_dot(wc, X);
            px = lane_dot(wx, X);
        }
        pb = wave_sum(pb);
        pc = wave_sum(pc);
        px = wave_sum(px);
        if (lane == 0)
            conv_step(pb, pc, px, a.conv_w + ch * 3, a.state + ch * 2, a.y + ch);
    }
}

// Attention projections q (dim rows), k and v (hdkv rows each) of the normed
// input, written raw to qkv[0..dim+2*hdkv).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_qkv(const QkvArgs a)
{
    if (a.st->halt)
        return;
    extern __shared__ float smem[];
    float *xs = smem;
    float *red = smem + a.dim;
    stage_x(a.src, xs, a.dim, a.st, red);
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.wq.nb;
    LaneX X;
    if (active)
        load_lanex(X, xs, b, c);
    else
        zero_lanex(X);
    const uint32_t total = a.dim + 2 * a.hdkv;
    for (uint32_t r = blockIdx.x * 4 + wave; r < total; r += gridDim.x * 4) {
        float p = 0.f;
        if (active) {
            if (r < a.dim)
                p = lane_dot(load_lane(a.wq, r, b, c), X);
            else if (r < a.dim + a.hdkv)
                p = lane_dot(load_lane(a.wk, r - a.dim, b, c), X);
            else
                p = lane_dot(load_lane(a.wv, r - a.dim - a.hdkv, b, c), X);
        }
        p = wave_sum(p);
        if (lane == 0)
            a.qkv[r] = p;
    }
}

// Per-head RMSNorm then NEOX RoPE of one 64-wide head held one value per lane
// (lfm.rs:270-286 then 248-267): v *= inv * w[d]; pairs (d, d+32) rotated by
// theta = pos * tscale^(d%32) with tscale^p by square-and-multiply.
__device__ __forceinline__ float f32_powi(float a, int b)
{
    float r = 1.0f;
    for (;;) {
        if (b & 1)
            r *= a;
        b /= 2;
        if (b == 0)
            break;
        a *= a;
    }
    return r;
}

__device__ __forceinline__ float head_norm_rope(float v, const float *w, float eps, float tscale,
                                                uint32_t pos, uint32_t d)
{
    const float ss = wave_sum(v * v);
    const float inv = 1.0f / sqrtf(ss / 64.0f + eps);
    v *= inv * w[d];
    const float other = __shfl_xor(v, 32, 64);
    const uint32_t p = d & 31;
    const float theta = (float)pos * f32_powi(tscale, (int)p);
    const float sn = sinf(theta), cs = cosf(theta);
    // lane d < 32 holds x0 (partner x1); lane d >= 32 holds x1 (partner x0)
    return d < 32 ? v * cs - other * sn : other * sn + v * cs;
}

// Split-K decode attention over the binary16 KV cache, one workgroup per
// (position chunk of 128, kv head); the G = heads/kv query heads of a kv head
// share the K/V reads.  The workgroup holding the current position also
// normalizes, rotates, rounds and stores the new K/V row.  Partials
// (max, sum, o[64]) are merged by the last workgroup of each kv head.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_attn(const AttnArgs a)
{
    if (a.st->halt)
        return;
    const uint32_t p = a.st->pos;
    const uint32_t kh = blockIdx.y, chunk = blockIdx.x;
    const uint32_t t0 = chunk * ATT_CH;
    if (t0 > p)
        return;
    const uint32_t nact = p / ATT_CH + 1;
    const uint32_t G = a.heads / a.kv;
    const uint32_t nt = min((uint32_t)ATT_CH, p + 1 - t0);
    const bool cur = (chunk == nact - 1);
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t dim = a.heads * 64, hdkv = a.kv * 64;

    __shared__ float qr[4][64];
    __shared__ float knew[64], vnew[64];
    __shared__ __attribute__((aligned(16))) uint16_t Ks[ATT_CH * ATT_KROW];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[ATT_CH * 64];
    __shared__ float sc[4][ATT_CH];
    __shared__ float stat[4][2];
    __shared__ uint32_t s_last;

    if (wave < G) {
        const float v = a.qkv[(kh * G + wave) * 64 + lane];
        qr[wave][lane] = head_norm_rope(v, a.q_norm, a.eps, a.tscale, p, lane);
    }
    if (cur && wave == 0) {
        const float kraw = a.qkv[dim + kh * 64 + lane];
        const float kr = head_norm_rope(kraw, a.k_norm, a.eps, a.tscale, p, lane);
        const uint16_t kb = float_to_half_bits(kr);
        const uint16_t vb = float_to_half_bits(a.qkv[dim + hdkv + kh * 64 + lane]);
        a.kcache[((size_t)kh * a.ctx + p) * 64 + lane] = kb;
        a.vcache[((size_t)kh * a.ctx + p) * 64 + lane] = vb;
        knew[lane] = half_bits_to_float(kb);
        vnew[lane] = half_bits_to_float(vb);
    }
    // K/V rows of this chunk -> LDS (16 B per thread per pass).
    const uint16_t *kg = a.kcache + ((size_t)kh * a.ctx + t0) * 64;
    const uint16_t *vg = a.vcache + ((size_t)kh * a.ctx + t0) * 64;
    for (uint32_t u = tid; u < nt * 8; u += WG_THREADS) {
        const uint32_t t = u >> 3, seg = u & 7;
        if (t0 + t != p) {
            *reinterpret_cast<uint4 *>(Ks + t * ATT_KROW + seg * 8) =
                *reinterpret_cast<const uint4 *>(kg + t * 64 + seg * 8);
            *reinterpret_cast<uint4 *>(Vs + t * 64 + seg * 8) =
                *reinterpret_cast<const uint4 *>(vg + t * 64 + seg * 8);
        }
    }
    __syncthreads();
    // scores: thread -> position t, heads 2*hp and 2*hp+1
    {
        const uint32_t t = tid & (ATT_CH - 1), hp = tid >> 7;
        const bool isnew = (t0 + t == p);
        for (uint32_t hh = 2 * hp; hh < 2 * hp + 2; ++hh) {
            if (hh >= G)
                break;
            float s = -INFINITY;
            if (t < nt) {
                float acc = 0.f;
                if (isnew) {
                    for (int d = 0; d < 64; ++d)
                        acc += qr[hh][d] * knew[d];
                } else {
#pragma unroll
                    for (int d8 = 0; d8 < 8; ++d8) {
                        const uint4 kv8 = *reinterpret_cast<const uint4 *>(Ks + t * ATT_KROW + d8 * 8);
                        const uint32_t w4[4] = {kv8.x, kv8.y, kv8.z, kv8.w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            acc += qr[hh][d8 * 8 + 2 * j] * half_bits_to_float(w4[j] & 0xFFFFu);
                            acc += qr[hh][d8 * 8 + 2 * j + 1] * half_bits_to_float(w4[j] >> 16);
                        }
                    }
                }
                s = acc * a.scale;
            }
            sc[hh][t] = s;
        }
    }
    __syncthreads();
    if (wave < G) {
        const float s0 = sc[wave][lane], s1 = sc[wave][lane + 64];
        const float m = wave_max(fmaxf(s0, s1));
        const float e0 = expf(s0 - m), e1 = expf(s1 - m);
        sc[wave][lane] = e0;
        sc[wave][lane + 64] = e1;
        const float l = wave_sum(e0 + e1);
        if (lane == 0) {
            stat[wave][0] = m;
            stat[wave][1] = l;
        }
    }
    __syncthreads();
    const uint32_t hh = tid >> 6, d = tid & 63;
    float *part = a.part + (((size_t)kh * a.nchunk + chunk) * 4 + hh) * 66;
    if (hh < G) {
        float acc = 0.f;
        for (uint32_t t = 0; t < nt; ++t) {
            const float vv = (t0 + t == p) ? vnew[d] : half_bits_to_float(Vs[t * 64 + d]);
            acc += sc[hh][t] * vv;
        }
        part[2 + d] = acc;
        if (d == 0) {
            part[0] = stat[hh][0];
            part[1] = stat[hh][1];
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.st->counters[LFM_CNT_ATTN + kh], 1u);
        s_last = (prev == nact - 1);
    }
    __syncthreads();
    if (!s_last)
        return;
    __threadfence();
    if (hh < G) {
        const float *pb = a.part + ((size_t)kh * a.nchunk * 4 + hh) * 66;
        float M = -INFINITY;
        for (uint32_t cc = 0; cc < nact; ++cc)
            M = fmaxf(M, __builtin_nontemporal_load(pb + (size_t)cc * 4 * 66));
        float acc = 0.f, L = 0.f;
        for (uint32_t cc = 0; cc < nact; ++cc) {
            const float *pc = pb + (size_t)cc * 4 * 66;
            const float f = expf(__builtin_nontemporal_load(pc) - M);
            L += f * __builtin_nontemporal_load(pc + 1);
            acc += f * __builtin_nontemporal_load(pc + 2 + d);
        }
        a.out[(kh * G + hh) * 64 + d] = acc / L;
    }
    if (tid == 0)
        a.st->counters[LFM_CNT_ATTN + kh] = 0;
}

// MoE router (lfm.rs:599-637): logits = W_r h (f32), then the last workgroup
// takes sigmoid probabilities, score = p + bias, the top n_used by score with
// ties to the lower id (max score, then min id), weights p / max(sum, 2^-14).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_router(const RouterArgs a)
{
    if (a.st->halt)
        return;
    extern __shared__ float smem[];
    float *xs = smem;
    float *red = smem + a.dim;
    __shared__ uint32_t s_last;
    stage_x(a.src, xs, a.dim, a.st, red);
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t e = blockIdx.x * 4 + wave;
    if (e < a.n_expert) {
        const float *w = a.w + (size_t)e * a.dim;
        float acc = 0.f;
        for (uint32_t k = lane * 4; k < a.dim; k += 256) {
            const float4 wv = *reinterpret_cast<const float4 *>(w + k);
            acc += wv.x * xs[k] + wv.y * xs[k + 1] + wv.z * xs[k + 2] + wv.w * xs[k + 3];
        }
        acc = wave_sum(acc);
        if (lane == 0)
            a.logits[e] = acc;
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.st->counters[LFM_CNT_ROUTER], 1u);
        s_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last)
        return;
    __threadfence();
    if (wave == 0) {
        float prob = 0.f, score = -INFINITY;
        if (lane < a.n_expert) {
            const float lg = __builtin_nontemporal_load(a.logits + lane);
            prob = 1.0f / (1.0f + expf(-lg));
            score = prob + a.bias[lane];
        }
        float psel[8];
        uint32_t ids[8];
        for (uint32_t r = 0; r < a.n_used; ++r) {
            const float best = wave_max(score);
            const uint32_t cand = (lane < a.n_expert && score == best) ? lane : 0xFFFFFFFFu;
            const uint32_t id = wave_min_u32(cand);
            ids[r] = id;
            psel[r] = __shfl(prob, (int)id, 64);
            if (lane == id)
                score = -INFINITY;
        }
        if (lane == 0) {
            float wsum = 0.f;
            for (uint32_t r = 0; r < a.n_used; ++r)
                wsum = wsum + psel[r];
            if (wsum < 6.103515625e-5f)
                wsum = 6.103515625e-5f;
            for (uint32_t r = 0; r < a.n_used; ++r) {
                a.sel[r] = ids[r];
                a.sel[8 + r] = __float_as_uint(psel[r] / wsum);
            }
            a.st->counters[LFM_CNT_ROUTER] = 0;
        }
    }
}

// sw = g / (1 + exp(-g)) * u with g = Wg h, u = Wu h (lfm.rs:578-582, 655-659).
// Routed: work item (rank, row) reads expert sel[rank]'s rows.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_gateup(const GateUpArgs a)
{
    if (a.st->halt)
        return;
    extern __shared__ float smem[];
    const uint32_t in_dim = a.wg.nb * 256;
    float *xs = smem;
    float *red = smem + in_dim;
    stage_x(a.src, xs, in_dim, a.st, red);
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.wg.nb;
    LaneX X;
    if (active)
        load_lanex(X, xs, b, c);
    else
        zero_lanex(X);
    const uint32_t nrank = a.sel ? a.n_used : 1;
    const uint32_t total = nrank * a.ff;
    for (uint32_t item = blockIdx.x * 4 + wave; item < total; item += gridDim.x * 4) {
        const uint32_t rank = item / a.ff, r = item - rank * a.ff;
        uint32_t row = a.sel ? a.sel[rank] * a.ff + r : r;
        if (row >= a.wg.rows) // an id outside the table (NaN router scores) reads expert 0
            row = r;
        float g = 0.f, u = 0.f;
        if (active) {
            const Lane lg = load_lane(a.wg, row, b, c);
            const Lane lu = load_lane(a.wu, row, b, c);
            g = lane_dot(lg, X);
            u = lane_dot(lu, X);
        }
        g = wave_sum(g);
        u = wave_sum(u);
        if (lane == 0)
            a.sw[item] = g / (1.0f + expf(-g)) * u;
    }
}

// Routed down projections and combine (lfm.rs:660-668, resident.rs:101-117):
// wave r computes d_r = (Wd[e_r] sw_r)[k]; then
// x[k] += ((((0 + d_0 w_0) + d_1 w_1) + d_2 w_2) + d_3 w_3)  (no contraction).
__device__ __forceinline__ float combine4(const float *dv, const float *wv, uint32_t n, float x)
{
#pragma clang fp contract(off)
    float s = 0.0f;
    for (uint32_t r = 0; r < n; ++r)
        s = s + dv[r] * wv[r];
    return x + s;
}

extern "C" __global__ __launch_bounds__(WG_THREADS) void k_moe_down(const MoeDownArgs a)
{
    if (a.st->halt)
        return;
    __shared__ float red[2][4];
    __shared__ float wsel[4];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.wd.nb && wave < a.n_used;
    uint32_t e = a.sel[wave < a.n_used ? wave : 0];
    if ((size_t)e * a.dim + a.dim > a.wd.rows) // id outside the table (NaN scores): expert 0
        e = 0;
    if (tid < 4)
        wsel[tid] = tid < a.n_used ? __uint_as_float(a.sel[8 + tid]) : 0.f;
    LaneX X;
    if (active)
        load_lanex(X, a.sw + (size_t)wave * a.ff, b, c);
    else
        zero_lanex(X);
    const uint32_t dim = a.dim;
    for (uint32_t k0 = blockIdx.x * 2; k0 < dim; k0 += gridDim.x * 2) {
        float p0 = 0.f, p1 = 0.f;
        if (active) {
            const Lane l0 = load_lane(a.wd, e * dim + k0, b, c);
            const bool two = k0 + 1 < dim;
            const Lane l1 = load_lane(a.wd, e * dim + (two ? k0 + 1 : k0), b, c);
            p0 = lane_dot(l0, X);
            p1 = lane_dot(l1, X);
        }
        p0 = wave_sum(p0);
        p1 = wave_sum(p1);
        if (lane == 0) {
            red[0][wave] = p0;
            red[1][wave] = p1;
        }
        __syncthreads();
        if (tid < 2 && k0 + tid < dim)
            a.x[k0 + tid] = combine4(red[tid], wsel, a.n_used, a.x[k0 + tid]);
        __syncthreads();
    }
}

// (value, index) reduction for greedy argmax (main.rs:112-141): the larger
// value wins; equal values keep the lower index; -inf is "no candidate" and
// NaN never wins; with no candidate the result index is 0.
__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float v, uint32_t i)
{
    if (v > bv || (v == bv && v > -INFINITY && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void amax_wave(float &bv, uint32_t &bi)
{
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, off, 64);
        amax_merge(bv, bi, ov, oi);
    }
}

// Final reduction of per-workgroup partials by the last workgroup.
__device__ void amax_final(const float *partial, uint32_t n, float &bv, uint32_t &bi,
                           float (*redv)[4], uint32_t (*redi)[4])
{
    const uint32_t tid = threadIdx.x;
    bv = -INFINITY;
    bi = 0;
    for (uint32_t i = tid; i < n; i += WG_THREADS)
        amax_merge(bv, bi, __builtin_nontemporal_load(partial + 2 * i),
                   __float_as_uint(__builtin_nontemporal_load(partial + 2 * i + 1)));
    amax_wave(bv, bi);
    if ((tid & 63) == 0) {
        (*redv)[tid >> 6] = bv;
        (*redi)[tid >> 6] = bi;
    }
    __syncthreads();
    bv = (*redv)[0];
    bi = (*redi)[0];
    for (int w = 1; w < 4; ++w)
        amax_merge(bv, bi, (*redv)[w], (*redi)[w]);
}

// Final RMSNorm + tied Q6_K head (lfm.rs:676-693) with the greedy argmax fused;
// the last workgroup stores the winner and, in a decode step, feeds it back
// (stops the loop at eos, main.rs:182-189).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_head(const HeadArgs a)
{
    if (a.st->halt)
        return;
    extern __shared__ float smem[];
    const uint32_t dim = a.emb.nb * 256;
    float *xs = smem;
    float *red = smem + dim;
    __shared__ float redv[4];
    __shared__ uint32_t redi[4];
    __shared__ uint32_t s_last;
    stage_x(a.src, xs, dim, a.st, red);
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.emb.nb;
    LaneX X;
    if (active)
        load_lanex(X, xs, b, c);
    else
        zero_lanex(X);
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (uint32_t r = blockIdx.x * 4 + wave; r < a.vocab; r += gridDim.x * 4) {
        float v = active ? lane_dot(load_lane(a.emb, r, b, c), X) : 0.f;
        v = wave_sum(v);
        if (lane == 0 && a.logits)
            a.logits[r] = v;
        amax_merge(bv, bi, v, r);
    }
    if (lane == 0) {
        redv[wave] = bv;
        redi[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        float v = redv[0];
        uint32_t i = redi[0];
        for (int w = 1; w < 4; ++w)
            amax_merge(v, i, redv[w], redi[w]);
        a.partial[2 * blockIdx.x] = v;
        a.partial[2 * blockIdx.x + 1] = __uint_as_float(i);
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.st->counters[LFM_CNT_HEAD], 1u);
        s_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last)
        return;
    __threadfence();
    __shared__ float fredv[4];
    __shared__ uint32_t fredi[4];
    float fv;
    uint32_t fi;
    amax_final(a.partial, gridDim.x, fv, fi, &fredv, &fredi);
    if (tid == 0) {
        if (!(fv > -INFINITY))
            fi = 0;
        DevState *st = a.st;
        st->last_token = fi;
        st->last_value = fv;
        if (a.advance) {
            if (fi == st->eos) {
                st->halt = 1;
            } else {
                a.out_tokens[st->step] = fi;
                st->step = st->step + 1;
                st->tok = fi;
                st->pos = st->pos + 1;
            }
        }
        st->counters[LFM_CNT_HEAD] = 0;
    }
}

// Prompt stepping for the layer-only graph: next prompt id, next position.
extern "C" __global__ void k_advance(const AdvanceArgs a)
{
    if (threadIdx.x != 0 || a.st->halt)
        return;
    DevState *st = a.st;
    const uint32_t cur = st->cursor + 1;
    st->cursor = cur;
    st->pos = st->pos + 1;
    if (cur < st->n_ids)
        st->tok = a.ids[cur];
}

// Bit-exact dequantization of a packed tensor (parity check of the layout).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_q6_dequant(const DequantArgs a)
{
    const size_t units = (size_t)a.w.rows * a.w.nb * 8;
    for (size_t u = (size_t)blockIdx.x * WG_THREADS + threadIdx.x; u < units;
         u += (size_t)gridDim.x * WG_THREADS) {
        const uint32_t c = (uint32_t)(u & 7);
        const size_t blk = u >> 3;
        const uint32_t row = (uint32_t)(blk / a.w.nb), b = (uint32_t)(blk % a.w.nb);
        float v[32];
        lane_dequant(load_lane(a.w, row, b, c), v);
        float *o = a.out + (size_t)row * a.in_dim;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                o[lane_pos(b, c, s, i)] = v[s * 8 + i];
    }
}

// Stand-alone greedy argmax of a device vector.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_argmax(const ArgmaxArgs a)
{
    __shared__ float redv[4];
    __shared__ uint32_t redi[4];
    __shared__ uint32_t s_last;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (uint32_t i = blockIdx.x * WG_THREADS + tid; i < a.n; i += gridDim.x * WG_THREADS)
        amax_merge(bv, bi, a.v[i], i);
    amax_wave(bv, bi);
    if (lane == 0) {
        redv[wave] = bv;
        redi[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        float v = redv[0];
        uint32_t i = redi[0];
        for (int w = 1; w < 4; ++w)
            amax_merge(v, i, redv[w], redi[w]);
        a.partial[2 * blockIdx.x] = v;
        a.partial[2 * blockIdx.x + 1] = __uint_as_float(i);
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&a.st->counters[LFM_CNT_ARGMAX], 1u);
        s_last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!s_last)
        return;
    __threadfence();
    __shared__ float fredv[4];
    __shared__ uint32_t fredi[4];
    float fv;
    uint32_t fi;
    amax_final(a.partial, gridDim.x, fv, fi, &fredv, &fredi);
    if (tid == 0) {
        if (!(fv > -INFINITY))
            fi = 0;
        a.st->last_token = fi;
        a.st->last_value = fv;
        a.st->counters[LFM_CNT_ARGMAX] = 0;
    }
}
