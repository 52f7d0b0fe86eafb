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
//                                 (fused: partial sums in the output projection, total in gate/up)
//   SwiGLU                        engine/src/lfm.rs:578-582, kernels.rs:543-550
//   expert combine                engine/src/lfm.rs:645-668, kernels/resident.rs:101-117
//   embedding                     engine/src/lfm.rs:310-320, kernels/resident.rs:7-18
//   argmax                        engine/src/main.rs:112-141, kernels/persistent.rs:11-53
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kargs.h"
#include "q6_device.h"
#include "wave_ops.h"

#define WG_THREADS 256
#define ATT_CH 128  // attention positions per workgroup
#define ATT_KROW 72 // LDS row stride of a K row, in halves (144 B: conflict-free 16-B reads)

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

// The step's halt flag, read with a vector load: waiting for it (vmcnt counts
// in issue order) then leaves the weight loads issued after it in flight,
// where a scalar load's wait would also hold back everything issued later.
__device__ __forceinline__ uint32_t load_halt(const DevState *st)
{
    return __hip_atomic_load(&st->halt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The wave's index in its workgroup as a wave-uniform value, so that row
// indices derived from it (and the tensor fields selected by them) stay in
// scalar registers.
__device__ __forceinline__ uint32_t wave_index()
{
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
}

// A zero held in a vector register that the compiler cannot see through.
// Added to a wave-uniform index it keeps that load on the vector memory path:
// a scalar load is waited for with the counter that also covers LDS, so the
// first LDS wait after it (the input staging) would wait for memory too.
__device__ __forceinline__ uint32_t vzero()
{
    uint32_t z;
    asm("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// Workgroup barrier with no memory fence: it orders instruction issue only
// (the loads before it are all issued before any load after it), and waits
// for no data.
__device__ __forceinline__ void issue_barrier()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Compiler-only fence placed between a kernel's issued loads and its halt
// check: without it the compiler sinks the (unconditional) loads below the
// early return, so they would wait for the flag.
__device__ __forceinline__ void keep_issued() { asm volatile("" ::: "memory"); }

// ------------------------------------------------------------ staged input
// The input vector of a decode matvec (n <= 2048 values) is staged once per
// workgroup in LDS: xs[k] = x[k] * w[k] with w the RMSNorm weight, or x[k].
// RMSNorm's scalar inv = 1 / sqrt(sum x^2 / n + eps) (lfm.rs:231-244) then
// multiplies each finished dot product: row = inv * (W (x . w)).  That keeps
// the reduction off the path of the weight loads, which every kernel issues
// before staging.
#define XS_MAX 2048
#ifndef ISSUE_ORDER
#define ISSUE_ORDER() issue_barrier()
#endif

struct XRaw {
    float4 x0, x1, w0, w1;
    uint32_t tok; // embedding input: DevState::tok, loaded first
};

// Issues the loads of this thread's 8 values (positions 8t .. 8t+7).  The
// decode kernels issue every load without a branch around it (indices clamped
// into range, unused results ignored): a load under a branch leaves the
// compiler's wait counts unknown at the join, after which waiting for one
// early load also waits for every load issued after it.  Threads past n and
// the embedding case (x_out is then the residual buffer) load stand-ins.
template <bool EMB = false>
__device__ __forceinline__ void x_issue(const XSrc &s, uint32_t n, const DevState *st, XRaw &r)
{
    if constexpr (EMB)
        r.tok = __hip_atomic_load(&st->tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t k = min(threadIdx.x * 8, n - 8);
    const float *xp = s.embed ? s.x_out : s.x;
    const float *wp = s.norm_w ? s.norm_w : xp;
    r.x0 = *reinterpret_cast<const float4 *>(xp + k);
    r.x1 = *reinterpret_cast<const float4 *>(xp + k + 4);
    r.w0 = *reinterpret_cast<const float4 *>(wp + k);
    r.w1 = *reinterpret_cast<const float4 *>(wp + k + 4);
}

// Writes the staged vector, synchronizes the workgroup (every thread must
// call it) and returns inv (1 without a norm).  For the first kernel of a step
// the vector is the dequantized embedding row DevState::tok (lfm.rs:310-320),
// built by wave 0; workgroup 0 also stores it as the residual x_out.
// EMB = false compiles the embedding case out (its loads sit under a branch,
// see x_issue); the kernels of a step's first layer have EMB = true variants.
template <int NW, bool EMB = false>
__device__ __forceinline__ float x_stage(const XSrc &s, uint32_t n, const DevState *st,
                                         const XRaw &r, float *xs, float *red)
{
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float ss = 0.f;
    const uint32_t k = tid * 8;
    float v[8] = {r.x0.x, r.x0.y, r.x0.z, r.x0.w, r.x1.x, r.x1.y, r.x1.z, r.x1.w};
    if constexpr (EMB) {
        // The step's input is the embedding row of DevState::tok (lfm.rs:310-320):
        // wave 0 dequantizes it into xs, then every thread takes its 8 values
        // from there as in the plain case (workgroup 0 also stores the residual).
        if (wave == 0) {
            const uint32_t row = (uint32_t)__builtin_amdgcn_readfirstlane((int)r.tok);
            const uint32_t b = lane >> 3, c = lane & 7;
            if (b < n / 256) {
                float e32[32];
                lane_dequant(load_lane(s.emb, row, b, c), e32);
#pragma unroll
                for (int s4 = 0; s4 < 4; ++s4)
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        xs[lane_pos(b, c, s4, i)] = e32[s4 * 8 + i];
            }
        }
        __syncthreads();
        if (k < n) {
            const float4 a = *reinterpret_cast<const float4 *>(xs + k);
            const float4 bb = *reinterpret_cast<const float4 *>(xs + k + 4);
            v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
            v[4] = bb.x, v[5] = bb.y, v[6] = bb.z, v[7] = bb.w;
            if (blockIdx.x == 0 && s.x_out != nullptr) {
                *reinterpret_cast<float4 *>(s.x_out + k) = a;
                *reinterpret_cast<float4 *>(s.x_out + k + 4) = bb;
            }
        }
    }
    if (k < n) {
        float o[8];
        if (s.norm_w) {
            const float w[8] = {r.w0.x, r.w0.y, r.w0.z, r.w0.w, r.w1.x, r.w1.y, r.w1.z, r.w1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ss += v[i] * v[i];
                o[i] = v[i] * w[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                o[i] = v[i];
        }
        *reinterpret_cast<float4 *>(xs + k) = make_float4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<float4 *>(xs + k + 4) = make_float4(o[4], o[5], o[6], o[7]);
    }
    if (s.norm_w) {
        ss = wave_sum(ss);
        if (lane == 0)
            red[wave] = ss;
    }
    __syncthreads();
    if (!s.norm_w)
        return 1.0f;
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
        tot += red[w];
    return 1.0f / sqrtf(tot / (float)n + s.eps);
}

// A lane's 32 staged values (zero for lanes past the row's blocks).
__device__ __forceinline__ void lanex_lds(LaneX &X, const float *xs, uint32_t b, uint32_t c,
                                          bool active)
{
    if (active)
        load_lanex(X, xs, b, c);
    else
        zero_lanex(X);
}
// Sums of two / three per-lane partials across the wave (results in every lane).
__device__ __forceinline__ void wave_sum2(float &a, float &b)
{
    a = wave_sum(a);
    b = wave_sum(b);
}

__device__ __forceinline__ void wave_sum3(float &a, float &b, float &c)
{
    a = wave_sum(a);
    b = wave_sum(b);
    c = wave_sum(c);
}

// One wave's work items are it = first + k*W (k = 0, 1, ...) below `total`;
// each item is NR Q6_K rows.  Kernels load G items, reduce them, load the
// next G; the first group's loads are issued before the input is staged.
// Items past `total` load the last item again (never used), so no load sits
// under a branch.
template <int NR> struct Item {
    Lane l[NR];
};

template <int NR, int G, typename LoadF>
__device__ __forceinline__ void fill_items(Item<NR> (&buf)[G], uint32_t it0, uint32_t W,
                                           uint32_t total, LoadF load)
{
#pragma unroll
    for (int g = 0; g < G; ++g)
        load(min(it0 + g * W, total - 1), buf[g]);
}

// A lane's share of a row with the block index clamped into the row: lanes
// past the row's blocks (b >= nb) re-read its last block, which the dot
// products then leave out.
template <bool StreamAll = false>
__device__ __forceinline__ Lane load_lane_c(const Q6T &t, uint32_t row, uint32_t b, uint32_t c)
{
    return load_lane<StreamAll>(t, row, min(b, t.nb - 1), c);
}
// Wave sum of N per-lane values at once (results in every lane).
template <int N> __device__ __forceinline__ void wave_sum_n(float *v)
{
    wave_sums<N>(v);
}

// Old values y[it0 + g*W] of the rows a wave updates in place (lanes with
// `on`; others get 0), issued together with the rows' weights.
template <int G>
__device__ __forceinline__ void residual_issue(float (&yold)[G], const float *y, uint32_t it0,
                                               uint32_t W, uint32_t rows)
{
#pragma unroll
    for (int g = 0; g < G; ++g)
        yold[g] = y[min(it0 + g * W, rows - 1) + vzero()];
}

// ------------------------------------------------------------------ kernels
// Q6_K matvec y = W x (mode 0) or y += W x (mode 1), rows of up to 8 blocks:
// one wave per row, G rows in flight per wave, input staged per workgroup.
template <int NW, int G>
__device__ __forceinline__ void q6_matvec_body(const MatvecArgs &a)
{
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[XS_MAX];
    __shared__ float red[NW];
    const uint32_t lane = threadIdx.x & 63, wave = wave_index();
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.w.nb;
    const uint32_t W = gridDim.x * NW, first = blockIdx.x * NW + wave, rows = a.w.rows;
    auto load = [&](uint32_t r, Item<1> &it) { it.l[0] = load_lane_c(a.w, r, b, c); };
    XRaw raw;
    x_issue(a.src, a.in_dim, a.st, raw);
    Item<1> buf[G];
    fill_items(buf, first, W, rows, load);
    // mode 1: the rows' old values are loaded with the weights, not after the dot
    float yold[G];
    residual_issue<G>(yold, a.y, first, W, rows);
    keep_issued();
    if (halted) // checked after the loads are issued (the flag's latency overlaps them)
        return;
    const float inv = x_stage<NW>(a.src, a.in_dim, a.st, raw, xs, red);
    LaneX X;
    lanex_lds(X, xs, b, c, active);
    for (uint32_t it0 = first; it0 < rows; it0 += G * W) {
        if (it0 != first) {
            fill_items(buf, it0, W, rows, load);
            residual_issue<G>(yold, a.y, it0, W, rows);
        }
        float p[G];
#pragma unroll
        for (int g = 0; g < G; ++g)
            p[g] = (active && it0 + g * W < rows) ? lane_dot(buf[g].l[0], X) : 0.f;
        wave_sum_n<G>(p);
        if (lane == 0)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint32_t r = it0 + g * W;
                if (r < rows)
                    a.y[r] = a.mode ? yold[g] + inv * p[g] : inv * p[g];
            }
    }
}

extern "C" __global__ __launch_bounds__(256) void k_q6_matvec4(const MatvecArgs a)
{
    q6_matvec_body<4, 1>(a);
}
extern "C" __global__ __launch_bounds__(1024) void k_q6_matvec16(const MatvecArgs a)
{
    q6_matvec_body<16, 1>(a);
}

// Output projection y += W x (mode 1) with the router's first stage
// (lfm.rs:599-607): one wave per row, ROUTE_ROWS rows per workgroup.  Wave w
// (row r) loads row r of the transposed router weights (the 32 experts' R[e][r],
// one 128-byte line) and w_norm[r] with its weights; once its y[r] is known,
// lane e < 32 forms R[e][r] * (y[r] * w_norm[r]) and lane 32 y[r]^2.  Lanes
// q < 8 of wave 0 then add the workgroup's rows in order for experts 4q..4q+3
// and store them as one float4 (quad-major rpart), lane 8 the y^2 sum (rss).
// Lane 0 also stores y[r] * w_norm[r] in xw, the gate/up kernel's input.  The
// grid is exactly rows / ROUTE_ROWS.
extern "C" __global__ __launch_bounds__(64 * ROUTE_ROWS) void k_q6_matvec_route(const MatvecRouteArgs ra)
{
    const MatvecArgs &a = ra.m;
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[XS_MAX];
    __shared__ float red[ROUTE_ROWS];
    __shared__ float part[ROUTE_ROWS][ROUTE_EXPERTS + 1];
    const uint32_t lane = threadIdx.x & 63, wave = wave_index();
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.w.nb;
    const uint32_t r = blockIdx.x * ROUTE_ROWS + wave;
    XRaw raw;
    x_issue(a.src, a.in_dim, a.st, raw);
    ISSUE_ORDER();
    const Lane w = load_lane_c(a.w, r, b, c);
    const float yold = a.y[r + vzero()];
    const float rwe = ra.rwt[(size_t)r * ROUTE_EXPERTS + (lane & (ROUTE_EXPERTS - 1))];
    const float nwr = ra.rnorm[r + vzero()];
    keep_issued();
    if (halted)
        return;
    const float inv = x_stage<ROUTE_ROWS>(a.src, a.in_dim, a.st, raw, xs, red);
    LaneX X;
    lanex_lds(X, xs, b, c, active);
    const float p = wave_sum(active ? lane_dot(w, X) : 0.f);
    const float v = yold + inv * p;
    if (lane == 0) {
        a.y[r] = v;
        ra.xw[r] = v * nwr;
    }
    if (lane < ROUTE_EXPERTS)
        part[wave][lane] = rwe * (v * nwr);
    else if (lane == ROUTE_EXPERTS)
        part[wave][lane] = v * v;
    __syncthreads();
    if (wave == 0 && lane < ROUTE_QUADS) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < ROUTE_ROWS; ++i) {
            acc.x += part[i][4 * lane + 0];
            acc.y += part[i][4 * lane + 1];
            acc.z += part[i][4 * lane + 2];
            acc.w += part[i][4 * lane + 3];
        }
        reinterpret_cast<float4 *>(ra.rpart)[lane * ROUTE_PARTS + blockIdx.x] = acc;
    } else if (wave == 0 && lane == ROUTE_QUADS) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < ROUTE_ROWS; ++i)
            acc += part[i][ROUTE_EXPERTS];
        ra.rss[blockIdx.x] = acc;
    }
}
// Q6_K matvec for rows longer than 8 blocks (dense FFN down, 7168 inputs):
// `ksplit` waves share a row (nbw blocks each); x staged in LDS; partials
// combined in wave order.
// Q6_K matvec for rows of 9..32 blocks (2304..8192 inputs): a workgroup of 16
// waves owns LONG_ROWS rows; wave w takes K-chunk kc = w % 4 (blocks
// kc*nbw .. +nbw, nbw = ceil(nb / 4) <= 8) of rows r0 + w/4 and r0 + w/4 + 4.
// The input is staged once per workgroup; the first row's weights are issued
// before the staging and the second row's after it (a full load queue would
// otherwise stall the waves before the staging barrier).  Per row
//   y = ((p0 + p1) + p2) + p3   (mode 0)   or   y += that   (mode 1).
extern "C" __global__ __launch_bounds__(1024) void k_q6_matvec_long(const MatvecArgs a)
{
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[4 * XS_MAX];
    __shared__ float psh[LONG_ROWS][4];
    const uint32_t tid = threadIdx.x, wave = wave_index(), lane = tid & 63;
    const uint32_t kc = wave & 3, slot = wave >> 2;
    const uint32_t bl = lane >> 3, c = lane & 7;
    const uint32_t nbw = (a.w.nb + 3) / 4, b = kc * nbw + bl;
    const bool active = bl < nbw && b < a.w.nb;
    const uint32_t rows = a.w.rows, r0 = blockIdx.x * LONG_ROWS;
    const uint32_t n = a.in_dim; // = nb * 256 <= 4 * XS_MAX
    const uint32_t i0 = tid * 4, i1 = i0 + 1024 * 4;
    const float4 xv0 = *reinterpret_cast<const float4 *>(a.src.x + min(i0, n - 4));
    const float4 xv1 = *reinterpret_cast<const float4 *>(a.src.x + min(i1, n - 4));
    const uint32_t ry = min(r0 + (tid & (LONG_ROWS - 1)), rows - 1);
    const float yold = a.y[ry];
    const uint32_t bb = min(b, a.w.nb - 1);
    Item<1> buf[2];
    buf[0].l[0] = load_lane(a.w, min(r0 + slot, rows - 1), bb, c);
    keep_issued();
    if (halted)
        return;
    if (i0 < n)
        *reinterpret_cast<float4 *>(xs + i0) = xv0;
    if (i1 < n)
        *reinterpret_cast<float4 *>(xs + i1) = xv1;
    __syncthreads();
    buf[1].l[0] = load_lane(a.w, min(r0 + slot + 4, rows - 1), bb, c);
    LaneX X;
    lanex_lds(X, xs, b, c, active);
    float p[2];
#pragma unroll
    for (int g = 0; g < 2; ++g)
        p[g] = active ? lane_dot(buf[g].l[0], X) : 0.f;
    wave_sum_n<2>(p);
    if (lane == 0) {
        psh[slot][kc] = p[0];
        psh[slot + 4][kc] = p[1];
    }
    __syncthreads();
    if (tid < LONG_ROWS && r0 + tid < rows) {
        const float s = ((psh[tid][0] + psh[tid][1]) + psh[tid][2]) + psh[tid][3];
        a.y[r0 + tid] = a.mode ? yold + s : s;
    }
}

// Short-conv block, decode (lfm.rs:450-533 for n = 1): the wave of channel ch
// computes in_proj rows B[ch], C[ch], X[ch] of the normed input, then
//   bx = B*X; co = ((0 + s0*w0) + s1*w1) + bx*w2; y = C*co; state = (s1, bx)
// in the reference's operation order with no contraction.
// A channel's conv weights and state, loaded with its in_proj rows.
struct ConvCh {
    float w0, w1, w2, s0, s1;
};

__device__ __forceinline__ ConvCh conv_ch_load(const ConvInprojArgs &a, uint32_t ch)
{
    const uint32_t k = min(ch, a.dim - 1) + vzero();
    return ConvCh{a.conv_w[k * 3], a.conv_w[k * 3 + 1], a.conv_w[k * 3 + 2], a.state[k * 2],
                  a.state[k * 2 + 1]};
}

__device__ __forceinline__ void conv_step(float B, float C, float Xv, const ConvCh v, float *s2,
                                          float *y)
{
#pragma clang fp contract(off)
    const float bx = B * Xv;
    float co = 0.0f;
    co = co + v.s0 * v.w0;
    co = co + v.s1 * v.w1;
    co = co + bx * v.w2;
    *y = C * co;
    s2[0] = v.s1;
    s2[1] = bx;
}

// in_proj rows B[ch], C[ch], X[ch] of channel ch form one work item.
template <int NW, int G, bool EMB>
__device__ __forceinline__ void conv_inproj_body(const ConvInprojArgs &a)
{
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[XS_MAX];
    __shared__ float red[NW];
    const uint32_t lane = threadIdx.x & 63, wave = wave_index();
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.w.nb;
    const uint32_t dim = a.dim, W = gridDim.x * NW, first = blockIdx.x * NW + wave;
    auto load = [&](uint32_t ch, Item<3> &it) {
        it.l[0] = load_lane_c(a.w, ch, b, c);
        it.l[1] = load_lane_c(a.w, dim + ch, b, c);
        it.l[2] = load_lane_c(a.w, 2 * dim + ch, b, c);
    };
    XRaw raw;
    x_issue<EMB>(a.src, dim, a.st, raw);
    Item<3> buf[G];
    fill_items(buf, first, W, dim, load);
    ConvCh cv[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
        cv[g] = conv_ch_load(a, first + g * W);
    keep_issued();
    if (halted)
        return;
    const float inv = x_stage<NW, EMB>(a.src, dim, a.st, raw, xs, red);
    LaneX X;
    lanex_lds(X, xs, b, c, active);
    for (uint32_t it0 = first; it0 < dim; it0 += G * W) {
        if (it0 != first) {
            fill_items(buf, it0, W, dim, load);
#pragma unroll
            for (int g = 0; g < G; ++g)
                cv[g] = conv_ch_load(a, it0 + g * W);
        }
        float p[3 * G];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 3; ++j)
                p[3 * g + j] = (active && it0 + g * W < dim) ? lane_dot(buf[g].l[j], X) : 0.f;
        wave_sum_n<3 * G>(p);
        if (lane == 0)
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const uint32_t ch = it0 + g * W;
                if (ch < dim)
                    conv_step(inv * p[3 * g], inv * p[3 * g + 1], inv * p[3 * g + 2], cv[g],
                              a.state + ch * 2, a.y + ch);
            }
    }
}

extern "C" __global__ __launch_bounds__(256) void k_conv_inproj4(const ConvInprojArgs a)
{
    conv_inproj_body<4, 1, false>(a);
}
extern "C" __global__ __launch_bounds__(1024) void k_conv_inproj16(const ConvInprojArgs a)
{
    conv_inproj_body<16, 1, false>(a);
}
// First layer of a step: the input is the token's embedding row.
extern "C" __global__ __launch_bounds__(256) void k_conv_inproj4e(const ConvInprojArgs a)
{
    conv_inproj_body<4, 1, true>(a);
}
extern "C" __global__ __launch_bounds__(1024) void k_conv_inproj16e(const ConvInprojArgs a)
{
    conv_inproj_body<16, 1, true>(a);
}

// ------------------------------------------------------------ in-kernel handoff
// A fused kernel hands a vector from one phase to the next through tagged
// entries: the value's bits and a tag in one 64-bit word, stored and polled
// with agent-scope atomics, which are coherent across the XCDs' L2 caches
// without a cache flush.  The tag names the step generation (DevState::gen,
// advanced by the last kernel of every step) and the phase, so entries left by
// an earlier step or another phase never match and nothing is reset between
// graph replays; zeroed entries never match (bit 31 is always set).
__device__ __forceinline__ uint32_t flow_tag(uint32_t gen, uint32_t phase)
{
    return 0x80000000u | ((gen & 0x7FFFFFu) << 8) | (phase & 0xFFu);
}

__device__ __forceinline__ void flow_put(unsigned long long *e, uint32_t i, float v, uint32_t tag)
{
    __hip_atomic_store(e + i, ((unsigned long long)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Every wait is bounded: after FLOW_SPIN_LIMIT polls (well over 0.1 s) the
// waiter sets DevState::fault and goes on with what it read, and every later
// wait of any workgroup sees the fault and stops waiting, so the grid always
// drains; the host reports the fault.
#define FLOW_SPIN_LIMIT (1u << 17)
#ifndef FLOW_SLEEP
#define FLOW_SLEEP 1 // s_sleep between polls (units of 64 clocks)
#endif

// Values of entries k .. k+7 once each carries `tag`.
__device__ __forceinline__ void flow_get8(const unsigned long long *e, uint32_t k, uint32_t tag,
                                          float (&v)[8], DevState *st)
{
    unsigned long long w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        w[i] = __hip_atomic_load(e + k + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (uint32_t spins = 0;; ++spins) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            ok = ok && (uint32_t)(w[i] >> 32) == tag;
        if (ok)
            break;
        if (spins >= FLOW_SPIN_LIMIT || __hip_atomic_load(&st->fault, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            __hip_atomic_store(&st->fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
        __builtin_amdgcn_s_sleep(FLOW_SLEEP);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if ((uint32_t)(w[i] >> 32) != tag)
                w[i] = __hip_atomic_load(e + k + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        v[i] = __uint_as_float((uint32_t)w[i]);
}

// Short-conv mixer in one launch (lfm.rs:450-533 then the output projection and
// residual, with k_q6_matvec_route's router partial sums when ROUTE).  Wave w
// of workgroup g owns channel ch = 8g + w in phase A and output row r = ch in
// phase B; every value is computed as k_conv_inproj4 and k_q6_matvec_route /
// k_q6_matvec4 compute it (same staging sums, lane products, reductions and
// epilogues), so the results are bit-identical to the two-kernel chain.
// Phase A stages the normed input, forms the channel's B, C, X rows, the conv
// and the gate, and publishes the gated value as a tagged entry.  The
// output-projection row's weights are issued with phase A's at the start, so
// they arrive during phase A and the wait for all channels' values (phase B's
// input) instead of after it.
// The grid is dim / 8 workgroups, all co-resident (the host checks occupancy).
template <bool ROUTE>
__device__ __forceinline__ void conv_mixer_body(const ConvMixerArgs &a)
{
    constexpr int NW = 8;
    const ConvInprojArgs &c = a.in;
    const MatvecArgs &m = a.out.m;
    DevState *st = c.st;
    const uint32_t halted = load_halt(st);
    const uint32_t gen = __hip_atomic_load(&st->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __shared__ __attribute__((aligned(16))) float xs[XS_MAX];
    __shared__ __attribute__((aligned(16))) float gs[XS_MAX];
    __shared__ float red[NW];
    __shared__ float part[NW][ROUTE_EXPERTS + 1];
    const uint32_t lane = threadIdx.x & 63, wave = wave_index();
    const uint32_t b = lane >> 3, cl = lane & 7;
    const bool active = b < c.w.nb;
    const uint32_t dim = c.dim, ch = blockIdx.x * NW + wave, r = ch;
    // phase A's loads, then what phase B needs that phase A does not produce
    XRaw raw;
    x_issue(c.src, dim, st, raw);
    keep_issued(); // the input and its norm weight first: staging waits for them alone
    const Lane wb = load_lane_c(c.w, ch, b, cl);
    const Lane wc = load_lane_c(c.w, dim + ch, b, cl);
    const Lane wx = load_lane_c(c.w, 2 * dim + ch, b, cl);
    const ConvCh cv = conv_ch_load(c, ch);
    keep_issued(); // phase A's loads before phase B's: phase A waits for its own alone
    // phase B's weights: in flight through phase A and the handoff
    const Lane wo = load_lane_c(m.w, r, b, cl);
    const float yold = m.y[r + vzero()];
    float rwe = 0.f, nwr = 0.f;
    if constexpr (ROUTE) {
        rwe = a.out.rwt[(size_t)r * ROUTE_EXPERTS + (lane & (ROUTE_EXPERTS - 1))];
        nwr = a.out.rnorm[r + vzero()];
    }
    keep_issued();
    if (halted)
        return;
    const uint32_t tag = flow_tag(gen, a.phase);
    const float inv = x_stage<NW>(c.src, dim, st, raw, xs, red);
    LaneX X;
    lanex_lds(X, xs, b, cl, active);
    float p[3];
    p[0] = active ? lane_dot(wb, X) : 0.f;
    p[1] = active ? lane_dot(wc, X) : 0.f;
    p[2] = active ? lane_dot(wx, X) : 0.f;
    wave_sum_n<3>(p);
    if (lane == 0) {
        float g;
        conv_step(inv * p[0], inv * p[1], inv * p[2], cv, c.state + ch * 2, &g);
        flow_put(a.flow, ch, g, tag);
    }
    // phase B: every channel's gated value, staged (no norm: inv = 1)
    const uint32_t k = threadIdx.x * 8;
    if (k < dim) {
        float v[8];
        flow_get8(a.flow, k, tag, v, st);
        *reinterpret_cast<float4 *>(gs + k) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(gs + k + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    __syncthreads();
    LaneX G;
    lanex_lds(G, gs, b, cl, active);
    const float q = wave_sum(active ? lane_dot(wo, G) : 0.f);
    const float val = yold + 1.0f * q;
    if (lane == 0)
        m.y[r] = val;
    if constexpr (ROUTE) {
        if (lane == 0)
            a.out.xw[r] = val * nwr;
        if (lane < ROUTE_EXPERTS)
            part[wave][lane] = rwe * (val * nwr);
        else if (lane == ROUTE_EXPERTS)
            part[wave][lane] = val * val;
        __syncthreads();
        if (wave == 0 && lane < ROUTE_QUADS) {
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int i = 0; i < ROUTE_ROWS; ++i) {
                acc.x += part[i][4 * lane + 0];
                acc.y += part[i][4 * lane + 1];
                acc.z += part[i][4 * lane + 2];
                acc.w += part[i][4 * lane + 3];
            }
            reinterpret_cast<float4 *>(a.out.rpart)[lane * ROUTE_PARTS + blockIdx.x] = acc;
        } else if (wave == 0 && lane == ROUTE_QUADS) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < ROUTE_ROWS; ++i)
                acc += part[i][ROUTE_EXPERTS];
            a.out.rss[blockIdx.x] = acc;
        }
    }
}

extern "C" __global__ __launch_bounds__(512) void k_conv_mixer(const ConvMixerArgs a)
{
    conv_mixer_body<false>(a);
}
extern "C" __global__ __launch_bounds__(512) void k_conv_mixer_r(const ConvMixerArgs a)
{
    static_assert(ROUTE_ROWS == 8, "the fused router's partial sums cover one workgroup's 8 rows");
    conv_mixer_body<true>(a);
}

// Attention projections: rows of q (dim), k and v (hdkv each) of the normed
// input, written to qkv[0 .. dim + 2*hdkv).
__device__ __forceinline__ Lane qkv_lane(const QkvArgs &a, uint32_t r, uint32_t b, uint32_t c)
{
    // one load, from the tensor that holds row r (fields selected by value)
    const bool isq = r < a.dim, isk = !isq && r < a.dim + a.hdkv;
    Q6T t;
    t.base = isq ? a.wq.base : isk ? a.wk.base : a.wv.base;
    t.rows = isq ? a.wq.rows : isk ? a.wk.rows : a.wv.rows;
    t.nb = isq ? a.wq.nb : isk ? a.wk.nb : a.wv.nb;
    const uint32_t rr = isq ? r : isk ? r - a.dim : r - a.dim - a.hdkv;
    return load_lane_c(t, rr, b, c);
}

template <int NW, int G, bool EMB>
__device__ __forceinline__ void qkv_body(const QkvArgs &a)
{
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[XS_MAX];
    __shared__ float red[NW];
    const uint32_t lane = threadIdx.x & 63, wave = wave_index();
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.wq.nb;
    const uint32_t rows = a.dim + 2 * a.hdkv, W = gridDim.x * NW, first = blockIdx.x * NW + wave;
    auto load = [&](uint32_t r, Item<1> &it) { it.l[0] = qkv_lane(a, r, b, c); };
    XRaw raw;
    x_issue<EMB>(a.src, a.dim, a.st, raw);
    Item<1> buf[G];
    fill_items(buf, first, W, rows, load);
    keep_issued();
    if (halted)
        return;
    const float inv = x_stage<NW, EMB>(a.src, a.dim, a.st, raw, xs, red);
    LaneX X;
    lanex_lds(X, xs, b, c, active);
    for (uint32_t it0 = first; it0 < rows; it0 += G * W) {
        if (it0 != first)
            fill_items(buf, it0, W, rows, load);
        float p[G];
#pragma unroll
        for (int g = 0; g < G; ++g)
            p[g] = (active && it0 + g * W < rows) ? lane_dot(buf[g].l[0], X) : 0.f;
        wave_sum_n<G>(p);
        if (lane == 0)
#pragma unroll
            for (int g = 0; g < G; ++g)
                if (it0 + g * W < rows)
                    a.qkv[it0 + g * W] = inv * p[g];
    }
}

extern "C" __global__ __launch_bounds__(256) void k_qkv4(const QkvArgs a)
{
    qkv_body<4, 1, false>(a);
}
extern "C" __global__ __launch_bounds__(1024) void k_qkv16(const QkvArgs a)
{
    qkv_body<16, 1, false>(a);
}
extern "C" __global__ __launch_bounds__(256) void k_qkv4e(const QkvArgs a)
{
    qkv_body<4, 1, true>(a);
}
extern "C" __global__ __launch_bounds__(1024) void k_qkv16e(const QkvArgs a)
{
    qkv_body<16, 1, true>(a);
}
// Per-head RMSNorm then NEOX RoPE of one 64-wide head held one value per lane
// (lfm.rs:270-286 then 248-267): v *= inv * w[d]; pairs (d, d+32) rotated by
// theta = pos * tscale^(d%32).  cs_sn is the position's row of the (cos, sin)
// table the host fills at finalize with the reference's own arithmetic.
// The lane's norm weight w[d] and its (cos, sin) pair, loaded ahead of use.
struct HeadIn {
    float w, cs, sn;
};

__device__ __forceinline__ HeadIn head_in_load(const float *w, const float *cs_sn, uint32_t d)
{
    const uint32_t p = d & 31;
    return HeadIn{w[d], cs_sn[2 * p], cs_sn[2 * p + 1]};
}

__device__ __forceinline__ float head_norm_rope(float v, const HeadIn in, float eps, uint32_t d)
{
    const float ss = wave_sum(v * v);
    const float inv = 1.0f / sqrtf(ss / 64.0f + eps);
    v *= inv * in.w;
    const float2v vh = wave_halves(v);
    const float other = d < 32 ? vh[1] : vh[0];
    const float cs = in.cs, sn = in.sn;
    // lane d < 32 holds x0 (partner x1); lane d >= 32 holds x1 (partner x0)
    return d < 32 ? v * cs - other * sn : other * sn + v * cs;
}

// 16 bytes of one cached K row and of the V row: piece u of a chunk is row
// t0 + u/8, halves 8*(u%8) .. +8 (rows past the cache re-read its last row).
struct KvPiece {
    uint4 k, v;
};

__device__ __forceinline__ KvPiece kv_piece(const uint16_t *kg, const uint16_t *vg, uint32_t t0,
                                            uint32_t ctx, uint32_t u)
{
    const size_t off = (size_t)min(t0 + (u >> 3), ctx - 1) * 64 + (u & 7) * 8;
    return KvPiece{*reinterpret_cast<const uint4 *>(kg + off), *reinterpret_cast<const uint4 *>(vg + off)};
}

// Stores a piece in LDS: rows past the position as zeros (their weights are
// zero and the P.V loop runs over the whole chunk); the position's own row is
// left to the wave that computes it.
__device__ __forceinline__ void kv_stage(const KvPiece pc, uint16_t *Ks, uint16_t *Vs, uint32_t t0,
                                         uint32_t nt, uint32_t p, uint32_t u)
{
    const uint32_t t = u >> 3, seg = u & 7;
    if (t0 + t == p)
        return;
    const uint32_t m = t < nt ? 0xFFFFFFFFu : 0u; // per-word mask (no aggregate select)
    *reinterpret_cast<uint4 *>(Ks + t * ATT_KROW + seg * 8) =
        make_uint4(pc.k.x & m, pc.k.y & m, pc.k.z & m, pc.k.w & m);
    *reinterpret_cast<uint4 *>(Vs + t * 64 + seg * 8) =
        make_uint4(pc.v.x & m, pc.v.y & m, pc.v.z & m, pc.v.w & m);
}

// Split-K decode attention over the binary16 KV cache (lfm.rs:395-437): one
// workgroup per (chunk of 128 positions, kv head); the G = heads/kv query heads
// of a kv head share the K/V reads.  The workgroup holding the current position
// normalizes, rotates, rounds (RNE) and stores the new K/V row.  Each workgroup
// writes (max, sum, o[64]) per head; k_attn_merge combines the chunks.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_attn(const AttnArgs a)
{
    const uint32_t kh = blockIdx.y, chunk = blockIdx.x;
    const uint32_t t0 = chunk * ATT_CH;
    const uint32_t G = a.heads / a.kv;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t dim = a.heads * 64, hdkv = a.kv * 64;
    // Position and halt flag with vector loads; the chunk's K/V rows, q and the
    // new K/V values are issued before the position is known (rows past the
    // cache end re-read its last row and are never used), then the norm
    // weights and the position's RoPE row.
    const uint32_t pos_raw =
        __hip_atomic_load(&a.st->pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t halted = load_halt(a.st);
    static_assert(ATT_CH * 8 / WG_THREADS == 4, "four 16-B K and V pieces per thread");
    const uint16_t *kg = a.kcache + (size_t)kh * a.ctx * 64;
    const uint16_t *vg = a.vcache + (size_t)kh * a.ctx * 64;
    const KvPiece p0 = kv_piece(kg, vg, t0, a.ctx, tid);
    const KvPiece p1 = kv_piece(kg, vg, t0, a.ctx, tid + WG_THREADS);
    const KvPiece p2 = kv_piece(kg, vg, t0, a.ctx, tid + 2 * WG_THREADS);
    const KvPiece p3 = kv_piece(kg, vg, t0, a.ctx, tid + 3 * WG_THREADS);
    // q, k, v of the new position (clamped indices, no branch around the loads)
    const float qraw = a.qkv[(kh * G + min(wave, G - 1)) * 64 + lane];
    const float kraw = a.qkv[dim + kh * 64 + lane];
    const float vraw = a.qkv[dim + hdkv + kh * 64 + lane];
    // the position is waited for here, after every load above is issued
    uint32_t pos_v = pos_raw;
    asm volatile("" : "+v"(pos_v) : : "memory");
    const uint32_t p = (uint32_t)__builtin_amdgcn_readfirstlane((int)pos_v);
    const HeadIn hq = head_in_load(a.q_norm, a.rope + (size_t)p * 64, lane);
    const HeadIn hk = head_in_load(a.k_norm, a.rope + (size_t)p * 64, lane);
    keep_issued();
    if (halted || t0 > p)
        return;
    const uint32_t nact = p / ATT_CH + 1;
    const uint32_t nt = min((uint32_t)ATT_CH, p + 1 - t0);
    const bool cur = (chunk == nact - 1);

    __shared__ float qr[4][64];
    __shared__ __attribute__((aligned(16))) uint16_t Ks[ATT_CH * ATT_KROW];
    __shared__ __attribute__((aligned(16))) uint16_t Vs[ATT_CH * 64];
    __shared__ float sc[4][ATT_CH];
    __shared__ float stat[4][2];

    kv_stage(p0, Ks, Vs, t0, nt, p, tid);
    kv_stage(p1, Ks, Vs, t0, nt, p, tid + WG_THREADS);
    kv_stage(p2, Ks, Vs, t0, nt, p, tid + 2 * WG_THREADS);
    kv_stage(p3, Ks, Vs, t0, nt, p, tid + 3 * WG_THREADS);
    if (wave < G)
        qr[wave][lane] = head_norm_rope(qraw, hq, a.eps, lane);
    if (cur && wave == 0) {
        const float krot = head_norm_rope(kraw, hk, a.eps, lane);
        const uint16_t kb = float_to_half_bits(krot);
        const uint16_t vb = float_to_half_bits(vraw);
        a.kcache[((size_t)kh * a.ctx + p) * 64 + lane] = kb;
        a.vcache[((size_t)kh * a.ctx + p) * 64 + lane] = vb;
        Ks[(p - t0) * ATT_KROW + lane] = kb;
        Vs[(p - t0) * 64 + lane] = vb;
    }
    __syncthreads();
    // scores: thread -> position t, heads 2*hp and 2*hp+1
    {
        const uint32_t t = tid & (ATT_CH - 1), hp = tid >> 7;
        for (uint32_t hh = 2 * hp; hh < 2 * hp + 2; ++hh) {
            if (hh >= G)
                break;
            float s = -INFINITY;
            if (t < nt) {
                float acc = 0.f;
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
    // P.V: wave = head; lane (d4, tq) accumulates dims 4*d4 .. +3 over the
    // positions t = 4i + tq (a wave reads 512 contiguous bytes of V per step),
    // then the four position classes are summed across the lane quad.
    if (wave < G) {
        const uint32_t hh = wave, tq = lane & 3, d4 = lane >> 2;
        float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll 8
        for (uint32_t i = 0; i < ATT_CH / 4; ++i) {
            const uint32_t t = 4 * i + tq;
            const uint2 v = *reinterpret_cast<const uint2 *>(Vs + t * 64 + d4 * 4);
            const float pr = sc[hh][t];
            o0 += pr * half_bits_to_float(v.x & 0xFFFFu);
            o1 += pr * half_bits_to_float(v.x >> 16);
            o2 += pr * half_bits_to_float(v.y & 0xFFFFu);
            o3 += pr * half_bits_to_float(v.y >> 16);
        }
        o0 = quad_sum(o0), o1 = quad_sum(o1), o2 = quad_sum(o2), o3 = quad_sum(o3);
        float *part = a.part + (((size_t)kh * a.nchunk + chunk) * 4 + hh) * 66;
        if (tq == 0) {
            part[2 + 4 * d4] = o0;
            part[3 + 4 * d4] = o1;
            part[4 + 4 * d4] = o2;
            part[5 + 4 * d4] = o3;
        }
        if (lane == 0) {
            part[0] = stat[hh][0];
            part[1] = stat[hh][1];
        }
    }
}

// Combines the chunk partials of one head (workgroup (kv head, q head of the
// group)): out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c.  Four groups of
// 64 threads take every fourth chunk, all loads in flight at once, then the
// four partial merges are combined.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_attn_merge(const AttnMergeArgs a)
{
    if (a.st->halt)
        return;
    const uint32_t kh = blockIdx.x, hh = blockIdx.y;
    const uint32_t G = a.heads / a.kv;
    if (hh >= G)
        return;
    __shared__ float gm[4], gl[4], go[4][64];
    const uint32_t grp = threadIdx.x >> 6, d = threadIdx.x & 63;
    const uint32_t nact = a.st->pos / ATT_CH + 1;
    const float *pb = a.part + ((size_t)kh * a.nchunk * 4 + hh) * 66;
    float M = -INFINITY, acc = 0.f, L = 0.f;
    for (uint32_t c0 = grp; c0 < nact; c0 += 4 * 8) {
        float m[8], l[8], o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t cc = c0 + 4 * j;
            const bool ok = cc < nact;
            const float *pc = pb + (size_t)(ok ? cc : 0) * 4 * 66;
            m[j] = ok ? pc[0] : -INFINITY;
            l[j] = ok ? pc[1] : 0.f;
            o[j] = ok ? pc[2 + d] : 0.f;
        }
        float mn = M;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            mn = fmaxf(mn, m[j]);
        const float r = M > -INFINITY ? expf(M - mn) : 0.f;
        acc *= r;
        L *= r;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float f = m[j] > -INFINITY ? expf(m[j] - mn) : 0.f;
            L += f * l[j];
            acc += f * o[j];
        }
        M = mn;
    }
    if (d == 0) {
        gm[grp] = M;
        gl[grp] = L;
    }
    go[grp][d] = acc;
    __syncthreads();
    if (grp == 0) {
        const float mx = fmaxf(fmaxf(gm[0], gm[1]), fmaxf(gm[2], gm[3]));
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float f = gm[g] > -INFINITY ? expf(gm[g] - mx) : 0.f;
            num += f * go[g][d];
            den += f * gl[g];
        }
        a.out[(kh * G + hh) * 64 + d] = num / den;
    }
}

// MoE router logits W_r h (f32 weights [n_expert][dim], lfm.rs:599-607): one
// workgroup per expert; thread t covers inputs 8t .. 8t+7, so the workgroup
// also sums x^2 over the whole vector for the RMSNorm scale.
extern "C" __global__ __launch_bounds__(256) void k_router(const RouterArgs a)
{
    const uint32_t halted = load_halt(a.st);
    __shared__ float red[2][4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, e = blockIdx.x;
    const float *w = a.w + (size_t)e * a.dim;
    float ss = 0.f, acc = 0.f;
    for (uint32_t k = tid * 8; k < a.dim; k += 256 * 8) {
        const float4 x0 = *reinterpret_cast<const float4 *>(a.src.x + k);
        const float4 x1 = *reinterpret_cast<const float4 *>(a.src.x + k + 4);
        const float4 n0 = *reinterpret_cast<const float4 *>(a.src.norm_w + k);
        const float4 n1 = *reinterpret_cast<const float4 *>(a.src.norm_w + k + 4);
        const float4 w0 = *reinterpret_cast<const float4 *>(w + k);
        const float4 w1 = *reinterpret_cast<const float4 *>(w + k + 4);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const float nv[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ss += xv[i] * xv[i];
            acc += wv[i] * (xv[i] * nv[i]);
        }
    }
    keep_issued();
    if (halted)
        return;
    wave_sum2(ss, acc);
    if (lane == 0) {
        red[0][wave] = ss;
        red[1][wave] = acc;
    }
    __syncthreads();
    if (tid == 0) {
        const float tot = ((red[0][0] + red[0][1]) + red[0][2]) + red[0][3];
        const float dot = ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3];
        a.logits[e] = dot / sqrtf(tot / (float)a.dim + a.src.eps);
    }
}

// sw = g / (1 + exp(-g)) * u with g = Wg h, u = Wu h (lfm.rs:578-582, 655-659).
// FUSED: the router logits are the sums of the partials left by
// k_q6_matvec_route: wave w adds quad w's column (experts 4w..4w+3; each lane
// four rows, in row order, then a wave sum per expert) and every wave the x^2
// column; logit = dot / sqrt(sum x^2 / n + eps) as in k_router.  Its input needs no staging: each
// lane loads its 32 values of xw = x_new * w_norm (stored by k_q6_matvec_route)
// along with the partials, and 1 / rms comes from the x^2 column.
// Routed: work item (rank, row) reads expert ids[rank]'s rows.  The router
// logits are the first load; every wave computes the routing itself as soon as
// they arrive and issues its weight loads.  Workgroup 0 stores the routing (ids,
// weight bits) for the down projection.  Dense: the weight loads go out first.
template <int NW, int G, bool FUSED>
__device__ __forceinline__ void gateup_body(const GateUpArgs &a)
{
    static_assert(!FUSED || NW == ROUTE_QUADS, "fused router: one wave per quad of experts");
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[XS_MAX];
    __shared__ float red[NW];
    __shared__ float rsum[ROUTE_EXPERTS + 1];
    const uint32_t lane = threadIdx.x & 63, wave = wave_index();
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.wg.nb;
    const bool routed = FUSED || a.route.logits != nullptr;
    const uint32_t n = a.wg.nb * 256;
    const uint32_t ff = a.ff, total = (routed ? a.route.n_used : 1u) * ff;
    const uint32_t W = gridDim.x * NW, first = blockIdx.x * NW + wave;
    // router partial sums: lane l of wave w loads rows l + 64k (k < NK) of quad
    // w's column and float4 l of the x^2 column
    constexpr int NK = ROUTE_PARTS / 64;
    static_assert(ROUTE_PARTS == 256, "a wave holds the x^2 column as one float4 per lane");
    float4 pv[NK + 1];
    if constexpr (FUSED) {
        const float4 *pp = reinterpret_cast<const float4 *>(a.route.rpart) + wave * ROUTE_PARTS;
#pragma unroll
        for (int k = 0; k < NK; ++k)
            pv[k] = pp[lane + 64 * k];
        pv[NK] = reinterpret_cast<const float4 *>(a.route.rss)[lane];
    }
    RouteIn rin = route_load_all(a.route, a.src.x_out ? a.src.x_out : a.src.x);
    XRaw raw;
    LaneX X;
    if constexpr (FUSED)
        load_lanex(X, a.route.xw, b, c); // n = 2048: every lane is active
    else
        x_issue(a.src, n, a.st, raw);
    if constexpr (FUSED) {
        float4 q = pv[0];
#pragma unroll
        for (int k = 1; k < NK; ++k) {
            q.x += pv[k].x;
            q.y += pv[k].y;
            q.z += pv[k].z;
            q.w += pv[k].w;
        }
        float f[5] = {q.x, q.y, q.z, q.w,
                      (pv[NK].x + pv[NK].y) + (pv[NK].z + pv[NK].w)};
        wave_sums<5>(f);
        if (lane == 0) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                rsum[4 * wave + c] = f[c];
            if (wave == 0)
                rsum[ROUTE_EXPERTS] = f[4];
        }
        __syncthreads();
        // logit = dot / sqrt(sum x^2 / n + eps), with the hardware reciprocal
        // square root (n is a power of two, so the scaling by 1/n is exact)
        rin.lg = rsum[min(lane, (uint32_t)ROUTE_EXPERTS - 1)] *
                 __builtin_amdgcn_rsqf(rsum[ROUTE_EXPERTS] * __builtin_amdgcn_rcpf((float)n) + a.src.eps);
    }
    Routed rt = {0, 0, 0, 0, 0.f, 0.f, 0.f, 0.f};
    auto load = [&](uint32_t it, Item<2> &buf) {
        const uint32_t rank = it / ff, r = it - rank * ff;
        const uint32_t row = routed ? rt.id(rank) * ff + r : r;
        buf.l[0] = load_lane_c(a.wg, row, b, c);
        buf.l[1] = load_lane_c(a.wu, row, b, c);
    };
    Item<2> buf[G];
    float inv;
    if (routed) {
        // The input (loaded with the router partials) has arrived by the time
        // the routing is known: stage it first, then issue the weights.  A
        // wave stalls while the CU's load queue is full, so staging after a
        // deep weight issue would hold back every dot product.
        rt = wave_route_ids(a.route, rin);
        if (blockIdx.x == 0 && wave == 0 && a.route.sel_out) {
            Routed rw = rt;
            route_normalize(rw, a.route.n_used);
            if (lane < 8) {
                a.route.sel_out[lane] = lane < 4 ? rw.id(lane) : 0u;
                a.route.sel_out[8 + lane] = lane < 4 ? __float_as_uint(rw.w(lane)) : 0u;
            }
            // the record's logits and the scores the picks were ranked by
            if (lane < a.route.n_expert) {
                a.route.sel_out[ROUTE_REC_LOGITS + lane] = __float_as_uint(rin.lg);
                a.route.sel_out[ROUTE_REC_SCORES + lane] = __float_as_uint(route_score(rin));
            }
        }
        if (halted)
            return;
        if constexpr (FUSED) // RMSNorm's 1 / rms from the partial sums of x^2
            inv = 1.0f / sqrtf(rsum[ROUTE_EXPERTS] / (float)n + a.src.eps);
        else
            inv = x_stage<NW>(a.src, n, a.st, raw, xs, red);
        fill_items(buf, first, W, total, load);
    } else {
        fill_items(buf, first, W, total, load);
        keep_issued();
        if (halted)
            return;
        inv = x_stage<NW>(a.src, n, a.st, raw, xs, red);
    }
    if constexpr (!FUSED)
        lanex_lds(X, xs, b, c, active);
    for (uint32_t it0 = first; it0 < total; it0 += G * W) {
        if (it0 != first)
            fill_items(buf, it0, W, total, load);
        float p[2 * G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const bool ok = active && it0 + g * W < total;
            p[2 * g] = ok ? lane_dot(buf[g].l[0], X) : 0.f;
            p[2 * g + 1] = ok ? lane_dot(buf[g].l[1], X) : 0.f;
        }
        wave_sum_n<2 * G>(p);
        if (lane == 0)
#pragma unroll
            for (int g = 0; g < G; ++g)
                if (it0 + g * W < total) {
                    const float gv = inv * p[2 * g], uv = inv * p[2 * g + 1];
                    a.sw[it0 + g * W] = gv / (1.0f + expf(-gv)) * uv;
                }
    }
}

extern "C" __global__ __launch_bounds__(256) void k_gateup4(const GateUpArgs a)
{
    gateup_body<4, 2, false>(a);
}
extern "C" __global__ __launch_bounds__(1024) void k_gateup16(const GateUpArgs a)
{
    gateup_body<16, 2, false>(a);
}
// Fused router: 8-wave workgroups (measured best against 4 and 16: half the
// per-workgroup partial-sum and input reads of 4 waves, while 16 leave CUs idle).
extern "C" __global__ __launch_bounds__(512) void k_gateup8f(const GateUpArgs a)
{
    gateup_body<8, 2, true>(a);
}

// Routed down projections and combine (lfm.rs:660-668, resident.rs:101-117).
// A workgroup of 16 waves owns DOWN_ROWS output rows: wave w computes rows
// k0 + w/4 and k0 + w/4 + 4 of the expert of rank w%4, from that rank's sw
// staged in LDS; then per row
//   x[k] += ((((0 + d_0 w_0) + d_1 w_1) + d_2 w_2) + d_3 w_3)  (no contraction).
// The routing comes from the gate/up kernel (ids, then weight bits).
__device__ __forceinline__ float combine(const float *dv, const float *wv, uint32_t n, float x)
{
#pragma clang fp contract(off)
    float s = 0.0f;
    for (uint32_t r = 0; r < n; ++r)
        s = s + dv[r] * wv[r];
    return x + s;
}

#define DOWN_ROWS 8
extern "C" __global__ __launch_bounds__(1024) void k_moe_down(const MoeDownArgs a)
{
    if (!a.route.sel_out)
        return;
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[4 * XS_MAX];
    __shared__ float dsh[DOWN_ROWS][4];
    __shared__ float wsh[4];
    const uint32_t tid = threadIdx.x, wave = wave_index(), lane = tid & 63;
    const uint32_t b = lane >> 3, c = lane & 7;
    const uint32_t rank = wave & 3, slot = wave >> 2;
    const uint32_t n_used = a.route.n_used, ff = a.ff, dim = a.dim;
    const bool active = b < a.wd.nb && rank < n_used;
    const uint32_t k0 = blockIdx.x * DOWN_ROWS;
    // Load order: the expert id (the weight addresses depend on it), then what
    // does not depend on it (sw, the routing weights, the residual rows this
    // workgroup updates), then the expert's weights.
    // Every load is issued without a branch (indices clamped, unused values
    // ignored) so that the wait for the id does not also wait for the rest.
    const uint32_t e = min(a.route.sel_out[rank], a.route.n_expert - 1);
    const uint32_t nsw = n_used * ff; // <= 4 * XS_MAX (n_used <= 4, ff <= 2048)
    const uint32_t i0 = tid * 4, i1 = i0 + 1024 * 4;
    const float4 sv0 = *reinterpret_cast<const float4 *>(a.sw + min(i0, nsw - 4));
    const float4 sv1 = *reinterpret_cast<const float4 *>(a.sw + min(i1, nsw - 4));
    const uint32_t wbits = a.route.sel_out[8 + (tid & 3)];
    const float xold = a.x[min(k0 + (tid & (DOWN_ROWS - 1)), dim - 1)];
    // First row's weights, then the staging of sw, then the second row: with
    // both rows issued first, the CU's full load queue stalls the waves before
    // they reach the staging barrier.
    Item<1> buf[2];
    buf[0].l[0] = load_lane_c(a.wd, e * dim + min(k0 + slot, dim - 1), b, c);
    keep_issued();
    if (halted)
        return;
    if (tid < 4)
        wsh[tid] = __uint_as_float(wbits);
    if (i0 < nsw)
        *reinterpret_cast<float4 *>(xs + i0) = sv0;
    if (i1 < nsw)
        *reinterpret_cast<float4 *>(xs + i1) = sv1;
    __syncthreads();
    buf[1].l[0] = load_lane_c(a.wd, e * dim + min(k0 + slot + 4, dim - 1), b, c);
    LaneX X;
    lanex_lds(X, xs + rank * ff, b, c, active);
    float p[2];
#pragma unroll
    for (int g = 0; g < 2; ++g)
        p[g] = (active && k0 + slot + 4 * g < dim) ? lane_dot(buf[g].l[0], X) : 0.f;
    wave_sum_n<2>(p);
    if (lane == 0) {
        dsh[slot][rank] = p[0];
        dsh[slot + 4][rank] = p[1];
    }
    __syncthreads();
    if (tid < DOWN_ROWS && k0 + tid < dim)
        a.x[k0 + tid] = combine(dsh[tid], wsh, n_used, xold);
}
// (value, index) merge for greedy argmax (main.rs:112-141): the larger value
// wins; equal values keep the lower index; -inf is "no candidate" and NaN
// never wins; with no candidate the index is 0.
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

// Workgroup-level merge of per-wave (value, index); result in thread 0.
template <int NW = 4> __device__ __forceinline__ void amax_block(float &bv, uint32_t &bi)
{
    __shared__ float rv[NW];
    __shared__ uint32_t ri[NW];
    const uint32_t tid = threadIdx.x;
    amax_wave(bv, bi);
    if ((tid & 63) == 0) {
        rv[tid >> 6] = bv;
        ri[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NW; ++w)
            amax_merge(bv, bi, rv[w], ri[w]);
    }
}

// Final RMSNorm + tied Q6_K head (lfm.rs:676-693): one wave per row, G rows
// in flight; each workgroup leaves its argmax (value, index) partial for
// k_argmax_final.
template <int NW, int G>
__device__ __forceinline__ void head_body(const HeadArgs &a)
{
    const uint32_t halted = load_halt(a.st);
    __shared__ __attribute__((aligned(16))) float xs[XS_MAX];
    __shared__ float red[NW];
    const uint32_t lane = threadIdx.x & 63, wave = wave_index();
    const uint32_t b = lane >> 3, c = lane & 7;
    const bool active = b < a.emb.nb;
    const uint32_t rows = a.vocab, W = gridDim.x * NW, first = blockIdx.x * NW + wave;
    auto load = [&](uint32_t r, Item<1> &it) { it.l[0] = load_lane_c<true>(a.emb, r, b, c); };
    XRaw raw;
    x_issue(a.src, a.emb.nb * 256, a.st, raw);
    Item<1> buf[G];
    fill_items(buf, first, W, rows, load);
    keep_issued();
    if (halted)
        return;
    const float inv = x_stage<NW>(a.src, a.emb.nb * 256, a.st, raw, xs, red);
    LaneX X;
    lanex_lds(X, xs, b, c, active);
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (uint32_t it0 = first; it0 < rows; it0 += G * W) {
        if (it0 != first)
            fill_items(buf, it0, W, rows, load);
        float p[G];
#pragma unroll
        for (int g = 0; g < G; ++g)
            p[g] = (active && it0 + g * W < rows) ? lane_dot(buf[g].l[0], X) : 0.f;
        wave_sum_n<G>(p);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const uint32_t r = it0 + g * W;
            if (r < rows) {
                const float v = inv * p[g];
                if (lane == 0)
                    a.logits[r] = v;
                amax_merge(bv, bi, v, r);
            }
        }
    }
    amax_block<NW>(bv, bi);
    if (threadIdx.x == 0) {
        a.partial[2 * blockIdx.x] = bv;
        a.partial[2 * blockIdx.x + 1] = __uint_as_float(bi);
    }
}

extern "C" __global__ __launch_bounds__(256) void k_head4(const HeadArgs a)
{
    head_body<4, 2>(a);
}
extern "C" __global__ __launch_bounds__(1024) void k_head16(const HeadArgs a)
{
    head_body<16, 2>(a);
}
// Per-workgroup argmax partials of a plain vector.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_argmax(const ArgmaxArgs a)
{
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (uint32_t i = blockIdx.x * WG_THREADS + threadIdx.x; i < a.n; i += gridDim.x * WG_THREADS)
        amax_merge(bv, bi, a.v[i], i);
    amax_block<>(bv, bi);
    if (threadIdx.x == 0) {
        a.partial[2 * blockIdx.x] = bv;
        a.partial[2 * blockIdx.x + 1] = __uint_as_float(bi);
    }
}

// Reduces the partials; in a decode step stores the token and feeds it back
// (stops the loop at eos, main.rs:182-189).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_argmax_final(const FinalArgs a)
{
    if (a.st->halt)
        return;
    float bv = -INFINITY;
    uint32_t bi = 0;
    for (uint32_t i0 = threadIdx.x; i0 < a.n_partial; i0 += 4 * WG_THREADS) {
        float v[4];
        uint32_t ix[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t i = i0 + j * WG_THREADS;
            v[j] = i < a.n_partial ? a.partial[2 * i] : -INFINITY;
            ix[j] = i < a.n_partial ? __float_as_uint(a.partial[2 * i + 1]) : 0u;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            amax_merge(bv, bi, v[j], ix[j]);
    }
    amax_block<>(bv, bi);
    if (threadIdx.x == 0) {
        if (!(bv > -INFINITY))
            bi = 0;
        DevState *st = a.st;
        st->last_token = bi;
        st->last_value = bv;
        st->gen = st->gen + 1;
        if (a.host) {
            a.host->value = bv;
            a.host->fault = st->fault;
            a.host->token = bi;
        }
        if (a.advance) {
            if (bi == st->eos) {
                st->halt = 1;
            } else {
                a.out_tokens[st->step] = bi;
                st->step = st->step + 1;
                st->tok = bi;
                st->pos = st->pos + 1;
            }
        }
    }
}

// Prompt stepping for the layer-only graph: next prompt id, next position.
extern "C" __global__ void k_advance(const AdvanceArgs a)
{
    if (threadIdx.x != 0 || a.st->halt)
        return;
    DevState *st = a.st;
    st->gen = st->gen + 1;
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

// Plain streaming copy dst = src in 16-byte units (grid-stride): the reference
// for the achievable HBM rate and the scale of the memory-traffic counters.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_copy(const CopyArgs a)
{
    const uint64_t stride = (uint64_t)gridDim.x * WG_THREADS;
    for (uint64_t i = (uint64_t)blockIdx.x * WG_THREADS + threadIdx.x; i < a.n16; i += stride)
        a.dst[i] = a.src[i];
}
