// lfm_prefill.hip -- gfx950 MFMA kernels of the multi-token (prefill) path.
//
// Prefill is the one place the LFM2 token loop is a dense contraction: every
// projection multiplies a Q6_K weight by T activation columns.  The GEMM here
// runs on the matrix cores (v_mfma_f32_32x32x16_f16):
//   * each wave decodes its weight rows in registers to binary16 values
//     sc * (q - 32), which are exact whenever |sc * (q - 32)| <= 2048 (and within
//     1/2 ulp otherwise), straight into the MFMA A operand;
//   * the super-block scale d is applied in fp32 by rescaling the accumulators
//     once per 256-wide block;
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
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

#define WG_THREADS 256
// Split an f32 into binary16 hi + lo with hi = fp16(x), lo = fp16(x - hi).
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// Sums over the S slices of split-K partials, in slice order: v = p_0, then
// v += p_s.  The loads of a batch of slices are all issued before the first add
// (indexes clamped into range, the extra values unused; the batch is the smallest
// of 1, 2, 4, 8 that covers S, or 8, or at most BMAX); a load-add loop waited for
// each slice in turn.  NV sums share the batches: value n of slice s is at p + s *
// step + off[n].
template <int NV, int B>
__device__ __forceinline__ void slice_sums_b(const float *p, size_t step, uint32_t S, const size_t (&off)[NV],
                                             float (&v)[NV])
{
    for (uint32_t s0 = 0; s0 < S; s0 += B) {
        float q[NV][B];
#pragma unroll
        for (int j = 0; j < B; ++j)
#pragma unroll
            for (int n = 0; n < NV; ++n)
                q[n][j] = p[(size_t)min(s0 + j, S - 1) * step + off[n]];
#pragma unroll
        for (int j = 0; j < B; ++j)
#pragma unroll
            for (int n = 0; n < NV; ++n)
                if (s0 + j < S)
                    v[n] = s0 + j == 0 ? q[n][j] : v[n] + q[n][j];
    }
}
template <int NV, int BMAX = 8>
__device__ __forceinline__ void slice_sums(const float *p, size_t step, uint32_t S, const size_t (&off)[NV],
                                           float (&v)[NV])
{
    if (S <= 1) // uniform
        slice_sums_b<NV, 1>(p, step, S, off, v);
    else if (S <= 2 || BMAX < 4)
        slice_sums_b<NV, 2>(p, step, S, off, v);
    else if (S <= 4 || BMAX < 8)
        slice_sums_b<NV, 4>(p, step, S, off, v);
    else
        slice_sums_b<NV, 8>(p, step, S, off, v);
}

// RMSNorm (optional) of T rows of x [T][K], then a binary16 hi/lo split of
// x / scale with scale = 2^(e - 14) for max|x| = m * 2^e (so |x / scale| < 2^14).
// One workgroup per token row; K is a multiple of 256 up to 8192 (the engine's
// widths).  Thread tid owns the 8-element pieces p = tid + 256 i of the row
// (elements 8p .. 8p + 7), kept in registers, so the row is read once with
// 16-byte loads and each piece's hi and lo are one 16-byte store in either
// layout (row-major, or the token-blocked one where a piece of a logical row is
// 16 contiguous bytes).
#define SPLIT_NP 4 // pieces per thread: K <= 256 * 8 * SPLIT_NP

// Pieces v of row t (np of them valid for this thread), RMS-normed here with the
// matching pieces nw of the norm weight when a.norm_w is set, split into hi / lo of
// v / scale (scale[t] written): into row t (SPLIT_ROWMAJOR) or into the nl logical
// rows L[j] of the token-blocked layout.
// The workgroup barriers of the split wait only for LDS: a routing wave's list
// atomics (route_self) stay in flight across them.
__device__ __forceinline__ void split_barrier()
{
    __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// first() runs before the reductions; rows(L) fills the logical rows L[0..n) and
// returns n, after them, just before the stores.
template <typename Mid, typename Rows>
__device__ __forceinline__ void split_pieces(const SplitArgs &a, uint32_t t, float (&v)[SPLIT_NP][8],
                                             const float (&nw)[SPLIT_NP][8], Mid &&first, Rows &&rows)
{
    first();
    const uint32_t tid = threadIdx.x, npc = a.K >> 3;
    __shared__ float red[4], redm[4];
    if (a.norm_w) { // uniform
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < SPLIT_NP; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                ss += v[i][j] * v[i][j];
        ss = wave_sum(ss);
        if ((tid & 63) == 0)
            red[tid >> 6] = ss;
        split_barrier();
        const float tot = ((red[0] + red[1]) + red[2]) + red[3];
        const float inv = 1.0f / sqrtf(tot / (float)a.K + a.eps);
#pragma unroll
        for (int i = 0; i < SPLIT_NP; ++i) {
            const uint32_t pc = tid + WG_THREADS * i;
            if (pc < npc) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    v[i][j] = v[i][j] * inv * nw[i][j];
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < SPLIT_NP; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            amax = fmaxf(amax, fabsf(v[i][j]));
    amax = wave_max(amax);
    if ((tid & 63) == 0)
        redm[tid >> 6] = amax;
    split_barrier();
    amax = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    int e = 0;
    if (amax > 0.f && amax <= 3.0e38f)
        frexpf(amax, &e);
    const float scale = amax > 0.f ? ldexpf(1.0f, e - 14) : 1.0f, rs = 1.0f / scale;
    if (tid == 0)
        a.scale[t] = scale;
    uint32_t L[4];
    const uint32_t nl = rows(L);
    if (a.bscale && a.mode != SPLIT_ROWMAJOR) { // uniform
        const uint32_t nh = a.K >> 7;
        for (uint32_t q = 0; q < nl; ++q) // uniform
            for (uint32_t h = tid; h < nh; h += WG_THREADS)
                a.bscale[(size_t)L[q] * nh + h] = scale;
    }
    half8 *hi = reinterpret_cast<half8 *>(a.hi), *lo = reinterpret_cast<half8 *>(a.lo);
#pragma unroll
    for (int i = 0; i < SPLIT_NP; ++i) {
        const uint32_t pc = tid + WG_THREADS * i;
        if (pc >= npc)
            continue;
        half8 h, l;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            _Float16 hh, ll;
            split_f16(v[i][j] * rs, hh, ll);
            h[j] = hh;
            l[j] = ll;
        }
        if (a.mode == SPLIT_ROWMAJOR) {
            hi[(size_t)t * npc + pc] = h;
            lo[(size_t)t * npc + pc] = l;
        } else {
            for (uint32_t q = 0; q < nl; ++q) { // uniform
                const size_t o = ((size_t)(L[q] >> 5) * npc + pc) * 32 + (L[q] & 31);
                hi[o] = h;
                lo[o] = l;
            }
        }
    }
}

// Row t of x plus the down projection's ranks, as k_reduce_combine forms it:
// d_r = sum of the cksplit slices in slice order, then x + ((0 + d_0 w_0) + d_1 w_1
// ...) over the used ranks (lfm.rs:645-668, no contraction); the new values are
// written back to cx.  v holds the row's pieces (thread tid: pieces tid + 256 i).
__device__ __forceinline__ void combine_pieces(const SplitArgs &a, uint32_t t, float (&v)[SPLIT_NP][8])
{
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x, npc = a.K >> 3;
    const size_t D = a.K, slice = (size_t)a.T * 4 * D;
    float w[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        w[r] = a.cwsel[(size_t)t * 4 + r];
#pragma unroll
    for (int i = 0; i < SPLIT_NP; ++i) {
        const uint32_t pc = tid + WG_THREADS * i;
        if (pc >= npc)
            continue;
        const float *pp = a.cpart + (size_t)t * 4 * D + 8 * pc;
        float d[4][8];
        for (uint32_t s0 = 0; s0 < a.cksplit; s0 += 2) { // two slices' loads at a time
            float4 q[2][4][2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        q[j][r][h] = *reinterpret_cast<const float4 *>(
                            pp + (size_t)min(s0 + j, a.cksplit - 1) * slice + r * D + 4 * h);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                if (s0 + j < a.cksplit) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float qq[8] = {q[j][r][0].x, q[j][r][0].y, q[j][r][0].z, q[j][r][0].w,
                                             q[j][r][1].x, q[j][r][1].y, q[j][r][1].z, q[j][r][1].w};
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            d[r][e] = s0 + j == 0 ? qq[e] : d[r][e] + qq[e];
                    }
                }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float sm = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (r < (int)a.cn_used)
                    sm = sm + d[r][e] * w[r];
            v[i][e] = v[i][e] + sm;
        }
        float *o = a.cx + (size_t)t * D + 8 * pc;
        *reinterpret_cast<float4 *>(o) = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
        *reinterpret_cast<float4 *>(o + 4) = make_float4(v[i][4], v[i][5], v[i][6], v[i][7]);
    }
}

// The logical rows of token t's expert slots (SPLIT_GROUPED with tok set): slot r
// of t (r < n_used) goes to expert e_r = sel[t][r] at index pos_r = the number of
// earlier tokens that selected e_r (k_route_group's token order), found by every
// thread i < T testing token i's selection with ballots.  The workgroup also
// writes its slots' list entries and pos; workgroup 0 writes the counts.
__device__ __forceinline__ uint32_t route_rows(const SplitArgs &a, uint32_t t, uint32_t (&L)[4])
{
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ uint32_t wc[4][4], hist[64];
    uint32_t mine[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        mine[r] = a.sel[(size_t)t * 4 + r];
    uint32_t ids[4] = {~0u, ~0u, ~0u, ~0u};
    if (tid < a.T) {
        const uint4 s4 = *reinterpret_cast<const uint4 *>(a.sel + (size_t)tid * 4);
        ids[0] = s4.x, ids[1] = s4.y, ids[2] = s4.z, ids[3] = s4.w;
    }
    for (uint32_t r = a.n_used; r < 4; ++r)
        ids[r] = ~0u;
    if (t == 0) { // uniform
        if (tid < 64)
            hist[tid] = 0;
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (ids[r] < 64)
                atomicAdd(&hist[ids[r]], 1u);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const bool hit = tid < t && (ids[0] == mine[r] || ids[1] == mine[r] || ids[2] == mine[r] || ids[3] == mine[r]);
        const uint64_t m = __ballot(hit);
        if (lane == 0)
            wc[wave][r] = (uint32_t)__popcll(m);
    }
    __syncthreads();
    if (t == 0 && tid < a.n_expert)
        a.counts[tid] = hist[tid];
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (r < (int)a.n_used) {
            const uint32_t pr = wc[0][r] + wc[1][r] + wc[2][r] + wc[3][r], e = mine[r];
            L[r] = e * a.rpe + pr;
            if (tid == 0) {
                a.tok[(size_t)e * a.list_stride + pr] = t;
                a.slot[(size_t)e * a.list_stride + pr] = t * 4 + r;
                a.pos[(size_t)t * 4 + r] = pr;
            }
        }
    return a.n_used;
}

// EXT: the small calls' extra duties (a pending combine, the expert lists), in a
// kernel of their own so that the plain split keeps its registers.
// Routes token t in wave 0 (as k_route_topk does from the router partials) and
// takes list indexes for its slots by atomic adds on counts: the picks go to
// ids[] at once, the atomics' results (pr, lanes < n_used of wave 0) are used
// only by route_self_rows, after the split's reductions, so that their round trip
// overlaps them.
// (wave 0: the loads of its router partial sums, issued with the row's)
__device__ __forceinline__ void route_self_load(const SplitArgs &a, uint32_t t, float (&dp)[8], float (&sp)[8])
{
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) { // wave 0
        const uint32_t e = min(lane, a.n_expert - 1);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint32_t bb = min((uint32_t)b, a.nparts - 1);
            dp[b] = a.rpart[((size_t)t * a.nparts + bb) * a.n_expert + e];
            sp[b] = a.rss[(size_t)t * a.nparts + bb];
        }
    }
}
__device__ __forceinline__ uint32_t route_self_issue(const SplitArgs &a, uint32_t t, const float (&dp)[8],
                                                     const float (&sp)[8], uint32_t *ids)
{
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    uint32_t pr = 0;
    if (tid < 64) { // wave 0
        Route r;
        r.logits = nullptr;
        r.bias = a.rbias;
        r.n_expert = a.n_expert;
        r.n_used = a.n_used;
        r.sel_out = nullptr;
        const uint32_t e = min(lane, a.n_expert - 1);
        float dot = 0.f, ss = 0.f;
#pragma unroll
        for (int b = 0; b < 8; ++b)
            if (b < (int)a.nparts) {
                dot = b == 0 ? dp[b] : dot + dp[b];
                ss = b == 0 ? sp[b] : ss + sp[b];
            }
        const RouteIn in{dot / sqrtf(ss / (float)a.K + a.eps), a.rbias ? a.rbias[e] : 0.f};
        const Routed rt = wave_route(r, in);
        if (a.logit_out && lane < a.n_expert)
            a.logit_out[(size_t)t * a.n_expert + lane] = in.lg;
        if (lane < 4) {
            const uint32_t id = rt.id(lane);
            a.sel_out[(size_t)t * 4 + lane] = id;
            a.wsel_out[(size_t)t * 4 + lane] = lane < a.n_used ? rt.w(lane) : 0.f;
            ids[lane] = id;
            if (lane < a.n_used)
                pr = atomicAdd(&a.counts[id], 1u);
        }
    }
    return pr;
}

// The list entries of the routed slots and their logical rows L (route_self_issue).
__device__ __forceinline__ uint32_t route_self_rows(const SplitArgs &a, uint32_t t, const uint32_t *ids,
                                                    uint32_t *pos, uint32_t pr, uint32_t (&L)[4])
{
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    if (tid < 64 && lane < a.n_used) {
        const uint32_t id = ids[lane];
        pos[lane] = pr;
        a.tok[(size_t)id * a.list_stride + pr] = t;
        a.slot[(size_t)id * a.list_stride + pr] = t * 4 + lane;
        a.pos[(size_t)t * 4 + lane] = pr;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (r < (int)a.n_used)
            L[r] = ids[r] * a.rpe + pos[r];
    return a.n_used;
}

template <bool NORM, bool EXT>
__device__ __forceinline__ void split_rows_body(const SplitArgs &a, uint32_t t)
{
    const uint32_t tid = threadIdx.x, npc = a.K >> 3;
    const float *x = a.x + (size_t)t * a.K;
    // the norm weight's pieces are loaded with the row's, not after the sum of squares
    float v[SPLIT_NP][8], nw[SPLIT_NP][8];
#pragma unroll
    for (int i = 0; i < SPLIT_NP; ++i) {
        const uint32_t pc = tid + WG_THREADS * i;
        float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0, n0 = x0, n1 = x0;
        if (pc < npc) {
            x0 = *reinterpret_cast<const float4 *>(x + 8 * pc);
            x1 = *reinterpret_cast<const float4 *>(x + 8 * pc + 4);
            if (NORM) {
                n0 = *reinterpret_cast<const float4 *>(a.norm_w + 8 * pc);
                n1 = *reinterpret_cast<const float4 *>(a.norm_w + 8 * pc + 4);
            }
        }
        v[i][0] = x0.x, v[i][1] = x0.y, v[i][2] = x0.z, v[i][3] = x0.w;
        v[i][4] = x1.x, v[i][5] = x1.y, v[i][6] = x1.z, v[i][7] = x1.w;
        nw[i][0] = n0.x, nw[i][1] = n0.y, nw[i][2] = n0.z, nw[i][3] = n0.w;
        nw[i][4] = n1.x, nw[i][5] = n1.y, nw[i][6] = n1.z, nw[i][7] = n1.w;
    }
    if (a.copy_src) // uniform: one float4 per thread of the first copy_n / 1024 rows' workgroups
        for (uint32_t u = t * WG_THREADS + tid; u < a.copy_n / 4; u += a.T * WG_THREADS)
            reinterpret_cast<float4 *>(a.copy_dst)[u] = reinterpret_cast<const float4 *>(a.copy_src)[u];
    if (EXT && a.cpart) // uniform
        combine_pieces(a, t, v);
    if (EXT && a.mode == SPLIT_GROUPED && a.tok && a.rpart) { // uniform
        // the partial sums' loads go out with the row's, the picks and the list
        // atomics before the split's reductions, the list entries after them: the
        // atomics' round trip overlaps the reductions
        __shared__ uint32_t rids[4], rpos[4];
        float dp[8], sp[8];
        route_self_load(a, t, dp, sp);
        uint32_t pr = 0;
        split_pieces(
            a, t, v, nw,
            [&]() {
                // the row's loads (and the partial sums) complete here, so that the
                // reductions' uses of the row wait for nothing issued later
                __builtin_amdgcn_s_waitcnt(0x0f70); // vmcnt(0)
                pr = route_self_issue(a, t, dp, sp, rids);
            },
            [&](uint32_t (&L)[4]) { return route_self_rows(a, t, rids, rpos, pr, L); });
        return;
    }
    uint32_t L[4] = {t, 0, 0, 0}, nl = 1;
    if (EXT && a.mode == SPLIT_GROUPED && a.tok) { // uniform
        nl = route_rows(a, t, L);
    } else if (a.mode == SPLIT_GROUPED) { // uniform
        nl = 0;
        for (uint32_t j = 0; j < a.spr; ++j) {
            const uint32_t s = t * a.spr + j;
            if ((s & 3) < a.n_used)
                L[nl++] = a.sel[s] * a.rpe + a.pos[s];
        }
    }
    split_pieces(a, t, v, nw, []() {}, [&](uint32_t (&Lo)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            Lo[i] = L[i];
        return nl;
    });
}

extern "C" __global__ __launch_bounds__(WG_THREADS) void k_split_rows(const SplitArgs a)
{
    const uint32_t t = blockIdx.x;
    if (t >= a.T)
        return;
    if (a.norm_w) // uniform
        split_rows_body<true, false>(a, t);
    else
        split_rows_body<false, false>(a, t);
}

extern "C" __global__ __launch_bounds__(WG_THREADS) void k_split_rows_ext(const SplitArgs a)
{
    const uint32_t t = blockIdx.x;
    if (t >= a.T)
        return;
    if (a.norm_w) // uniform
        split_rows_body<true, true>(a, t);
    else
        split_rows_body<false, true>(a, t);
}

// s_waitcnt immediate (gfx9 encoding): vector-memory count <= n, LDS/scalar count 0,
// export count unconstrained.
#define WAITCNT_VM_LGKM0(n) ((((n) & 15) | (((n) >> 4) << 14)) | (7 << 4))

#define TM 256 // weight rows per workgroup (4 waves of 64 rows)
#define TN 128 // token columns per workgroup (each wave covers all of them)
#define TK 64  // K elements per stage (a quarter Q6_K block)
#define GEMM_NTH 256

// Activation tiles are [token][64 halves] = 8 pieces of 16 B per token; piece p
// of token row r holds k-piece p ^ ((r >> 1) & 7), so the 16-B fragment reads of
// 16 consecutive tokens fall in distinct banks.
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t kp) { return r * TK + ((kp ^ ((r >> 1) & 7)) << 3); }

// Activation tiles reach LDS by 16-byte buffer loads (buffer_load_dwordx4 ... lds):
// lane l's 16 bytes at byte offset voff of the buffer behind rs land in unit l of
// the wave's 1 KB at dst.  Unlike global_load_lds, which the compiler's wait
// insertion counts as an access to two memories (after which any use of a loaded
// register waits for every outstanding load), a buffer load keeps the
// vector-memory counter in issue order.  The restrict-qualified LDS pointers of
// these helpers give the DMA and the fragment reads alias scopes, from which the
// compiler sees that reading one buffer need not wait for the load into the other.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t act_rsrc(const uint16_t *base)
{
    // raw buffer: stride 0, offsets below 2^31 bytes (the host bounds the
    // activation buffers), data format dword
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(base), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, _Float16 *__restrict__ dst)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)dst, 16, voff, 0, 0, 0);
}
// One stage of a large call's hi and lo tiles: piece v of this wave, at byte offset
// boff[v] + k of the hi / lo buffers, to 16-byte units 256 v + 64 wave + lane of
// the tile (one call site per buffer pair, so that the compiler's per-store wait
// slots are not exhausted).
template <int NJ>
__device__ __forceinline__ void lds_dma_stage(__amdgpu_buffer_rsrc_t rh, __amdgpu_buffer_rsrc_t rl, const uint32_t (&boff)[NJ],
                                              uint32_t k, uint32_t wave, _Float16 *__restrict__ bh,
                                              _Float16 *__restrict__ bl)
{
#pragma unroll
    for (int v = 0; v < NJ; ++v) {
        const uint32_t u0 = (256 * v + 64 * wave) * 8;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, (__attribute__((address_space(3))) void *)&bh[u0], 16, boff[v] + k, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (__attribute__((address_space(3))) void *)&bl[u0], 16, boff[v] + k, 0, 0, 0);
    }
}
// Keeps the loads on either side in program order (for counted waits that rely on
// loads retiring in issue order): a compiler memory barrier and a scheduling barrier.
__device__ __forceinline__ void issue_fence()
{
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}
// A small-call stage's eight B fragments: hi and lo of k-steps 0..3, 16 bytes at
// byte offsets 1024 kq (hi) and 4096 + 1024 kq (lo) from the lane's address.  Issued
// in one asm statement, so that the compiler's wait insertion, which cannot tell
// these reads from reads of the tiles in flight once more than eight tile loads are
// in the code, does not make them wait for those loads; lds_frags_wait completes
// them (the stage's tile itself has landed: the barrier before the stage follows a
// wait for it).
__device__ __forceinline__ void lds_frags_issue(uint32_t addr, half8 (&h)[4], half8 (&l)[4])
{
    asm volatile("ds_read_b128 %0, %8\n\t"
                 "ds_read_b128 %1, %8 offset:1024\n\t"
                 "ds_read_b128 %2, %8 offset:2048\n\t"
                 "ds_read_b128 %3, %8 offset:3072\n\t"
                 "ds_read_b128 %4, %8 offset:4096\n\t"
                 "ds_read_b128 %5, %8 offset:5120\n\t"
                 "ds_read_b128 %6, %8 offset:6144\n\t"
                 "ds_read_b128 %7, %8 offset:7168"
                 : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3]), "=&v"(l[0]), "=&v"(l[1]), "=&v"(l[2]),
                   "=&v"(l[3])
                 : "v"(addr));
}
__device__ __forceinline__ void lds_frags_wait(half8 (&h)[4], half8 (&l)[4])
{
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(h[0]), "+v"(h[1]), "+v"(h[2]), "+v"(h[3]), "+v"(l[0]), "+v"(l[1]), "+v"(l[2]), "+v"(l[3]));
}
// 32-bit LDS address of a __shared__ object
typedef float floatx4 __attribute__((ext_vector_type(4)));
// Stores v at LDS byte address waddr, then reads the 16 floats at raddr + 32 k
// (k < 4, 4 each) back, in order within the wave, and waits for them.
__device__ __forceinline__ void lds_rowf(uint32_t waddr, float v, uint32_t raddr, floatx4 (&f)[4])
{
    asm volatile("ds_write_b32 %4, %5\n\t"
                 "ds_read_b128 %0, %6\n\t"
                 "ds_read_b128 %1, %6 offset:32\n\t"
                 "ds_read_b128 %2, %6 offset:64\n\t"
                 "ds_read_b128 %3, %6 offset:96\n\t"
                 "s_waitcnt lgkmcnt(0)"
                 : "=&v"(f[0]), "=&v"(f[1]), "=&v"(f[2]), "=&v"(f[3])
                 : "v"(waddr), "v"(v), "v"(raddr));
}

__device__ __forceinline__ uint32_t lds_addr(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ __forceinline__ half8 lds_frag(const _Float16 *__restrict__ b, uint32_t off)
{
    return *reinterpret_cast<const half8 *>(b + off);
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
// Bytes 0, 1 (hi false) or 2, 3 of t, each a 6-bit code c in bits 2..7 -> the
// binary16 pair 256 + c: the byte permute puts 0x5C (exponent 8) above each byte.
__device__ __forceinline__ half2v codes256(uint32_t t, bool hi)
{
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(t, 0x5C5C5C5Cu, hi ? 0x01070006u : 0x01050004u));
}

// A lane's Q6_K bytes for one half block (128 weights) of one row: the chunks of
// its two l0 groups (chunk c of the half block covers l0 in [8c', 8c' + 8)), each
// 32 six-bit codes in six words (the tile copy's code form) and the 4 scales.
struct AChunk {
    uint4 ql; // code words X0 .. X3
    uint2 qh; // code words X4, X5
    uint32_t sc;
};

// Lane `lane` (row lane % 32 of the tile, chunk parity lane / 32) of tile-block tb
// of the Q6Tiles planes at wb (ntb tile-blocks): chunks 4h + p and 4h + 2 + p of
// its row, i.e. half h of the block (5 loads: ql 1 KB and qh 512 B contiguous per
// wave and chunk pair, both chunks' scale groups as one 8-byte load).  STREAM: the
// ql / qh bytes are read once per call (small calls), so they are loaded
// non-temporally and do not displace the activations from the caches.
template <bool STREAM = false>
__device__ __forceinline__ void load_tile_chunks(const uint8_t *wb, size_t ntb, size_t tb, uint32_t h,
                                                 uint32_t lane, AChunk (&A)[2])
{
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
        const uint32_t q = 2 * h + ch;
        const uint8_t *pl = wb + tb * TILE_QL + q * 1024 + lane * 16;
        const uint8_t *ph = wb + ntb * TILE_QL + tb * TILE_QH + q * 512 + lane * 8;
        if (STREAM) {
            const u32x4_t l = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(pl));
            const u32x2_t hh = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(ph));
            A[ch].ql = make_uint4(l.x, l.y, l.z, l.w);
            A[ch].qh = make_uint2(hh.x, hh.y);
        } else {
            A[ch].ql = *reinterpret_cast<const uint4 *>(pl);
            A[ch].qh = *reinterpret_cast<const uint2 *>(ph);
        }
    }
    const uint2 sc = *reinterpret_cast<const uint2 *>(wb + ntb * (TILE_QL + TILE_QH) + tb * TILE_SC + h * 256 +
                                                      (lane & 31) * 8);
    A[0].sc = sc.x;
    A[1].sc = sc.y;
}

// binary16 bits of d of row r of tile-block tb
__device__ __forceinline__ uint32_t tile_d(const uint8_t *wb, size_t ntb, size_t tb, uint32_t r)
{
    return reinterpret_cast<const uint16_t *>(wb + ntb * (TILE_QL + TILE_QH + TILE_SC) + tb * TILE_D)[r];
}

// The code words of one chunk half w (l = l0 + 4w + b, byte b) from its row-major
// plane words: A = ql[l], B = ql[l + 32], H = qh[l].  The Q6_K codes of sub-blocks
// 0..3 are (A & 15) | (H & 3) << 4, (B & 15) | (H >> 2 & 3) << 4, (A >> 4) | (H >> 4
// & 3) << 4 and (B >> 4) | (H >> 6) << 4 (the element order of q6k.rs's dequant);
// word s < 3 holds code s in bits 2..7 of each byte and bits 2s, 2s + 1 of code 3
// in bits 0..1.
__device__ __forceinline__ void code_words(uint32_t A, uint32_t B, uint32_t H, uint32_t (&X)[3])
{
    const uint32_t M4 = 0x0F0F0F0Fu, M2 = 0x30303030u, M1 = 0x03030303u;
    const uint32_t c0 = (A & M4) | ((H << 4) & M2), c1 = (B & M4) | ((H << 2) & M2);
    const uint32_t c2 = ((A >> 4) & M4) | (H & M2), c3 = ((B >> 4) & M4) | ((H >> 2) & M2);
    X[0] = (c0 << 2) | (c3 & M1);
    X[1] = (c1 << 2) | ((c3 >> 2) & M1);
    X[2] = (c2 << 2) | ((c3 >> 4) & M1);
}

// Row-major Q6_K planes -> Q6Tiles (the layout is described with the struct).
// Workgroup tb (64 lanes, lane l = 32 p + r) writes tile-block tb: rows past the
// slice's end are zero (d = 0: they contribute zero weights).
extern "C" __global__ __launch_bounds__(64) void k_q6_tile_pack(const TilePackArgs a)
{
    const uint32_t tb = blockIdx.x, l = threadIdx.x, p = l >> 5, r = l & 31;
    const uint32_t nb = a.src.nb, t = tb / nb, kb = tb - t * nb;
    const uint32_t g = t / a.gtiles, row = (t - g * a.gtiles) * 32 + r;
    const bool ok = row < a.group_rows;
    const size_t nblk = (size_t)a.src.rows * nb, ntb = (size_t)a.tiles * nb;
    const size_t blk = ((size_t)g * a.group_rows + (ok ? row : 0)) * nb + kb;
    const uint8_t *s = a.src.base;
    uint8_t *d = a.dst;
#pragma unroll
    for (uint32_t q = 0; q < 4; ++q) {
        const uint32_t c = 2 * q + p;
        const uint4 vl = ok ? *reinterpret_cast<const uint4 *>(s + blk * 128 + c * 16) : make_uint4(0, 0, 0, 0);
        const uint2 vh = ok ? *reinterpret_cast<const uint2 *>(s + nblk * 128 + blk * 64 + c * 8) : make_uint2(0, 0);
        uint32_t X0[3], X1[3]; // chunk halves w = 0, 1
        code_words(vl.x, vl.z, vh.x, X0);
        code_words(vl.y, vl.w, vh.y, X1);
        *reinterpret_cast<uint4 *>(d + tb * TILE_QL + q * 1024 + l * 16) = make_uint4(X0[0], X1[0], X0[1], X1[1]);
        *reinterpret_cast<uint2 *>(d + ntb * TILE_QL + tb * TILE_QH + q * 512 + l * 8) = make_uint2(X0[2], X1[2]);
    }
    // scales as sc + 128 (sc ^ 0x80), or 128 throughout when d is +-0
    const uint16_t vd = ok ? reinterpret_cast<const uint16_t *>(s + nblk * 208)[blk] : (uint16_t)0;
    const uint2 vs = ok ? *reinterpret_cast<const uint2 *>(s + nblk * 192 + blk * 16 + p * 8) : make_uint2(0, 0);
    const bool dz = (vd & 0x7FFFu) == 0;
    const uint2 vb = dz ? make_uint2(0x80808080u, 0x80808080u) : make_uint2(vs.x ^ 0x80808080u, vs.y ^ 0x80808080u);
    *reinterpret_cast<uint2 *>(d + ntb * (TILE_QL + TILE_QH) + tb * TILE_SC + p * 256 + r * 8) = vb;
    // a stored byte b = sc + 128 outside [64, 192] is a scale outside [-64, 64]
    bool wide = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t byte = ((i < 4 ? vb.x : vb.y) >> (8 * (i & 3))) & 0xFFu;
        wide = wide || byte < 64u || byte > 192u;
    }
    if (__ballot(wide) != 0 && l == 0)
        __hip_atomic_store(a.wide, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (p == 0)
        reinterpret_cast<uint16_t *>(d + ntb * (TILE_QL + TILE_QH + TILE_SC) + tb * TILE_D)[r] = vd;
}

// The scales of sub-blocks 2q and 2q + 1 of a chunk as binary16 (sc) and -288
// times them (bias): its scale bytes are sc + 128 (zero throughout a block whose d
// is zero), so the byte permute that forms 1024 + (sc + 128) and a subtraction of
// 1152 give sc exactly; 288 sc = 9 sc * 32 is exact too (|9 sc| <= 1152).
struct StageScales {
    half2v sc, bias;
};
__device__ __forceinline__ StageScales stage_scales(uint32_t sc, int q)
{
    const uint32_t v = __builtin_amdgcn_perm(sc, 0x64646464u, q ? 0x01070006u : 0x01050004u);
    const half2v s = __builtin_bit_cast(half2v, v) - (half2v){(_Float16)1152.0f, (_Float16)1152.0f};
    return {s, s * (half2v){(_Float16)-288.0f, (_Float16)-288.0f}};
}

// The split form of the stage's scales, for weights whose products sc (q6 - 32)
// can exceed 2048 in magnitude (a binary16 holds every integer up to 2048 only):
// sc = sh + sl with sh = sc & ~15 (a multiple of 16) and sl = sc & 15, formed from
// the stored byte b = sc + 128 as (b & 0xF0) - 128 and b & 15.  Both partial
// weights are exact binary16 values for every int8 scale: sh (q6 - 32) is 16
// times an integer of magnitude <= 256, and |sl (q6 - 32)| <= 480; so are the
// biases -288 sh (= -9 (sh / 16) 512) and -288 sl.
struct SplitScales {
    half2v sh, sl;
};
__device__ __forceinline__ SplitScales stage_scales_split(uint32_t sc, int q)
{
    const uint32_t sel = q ? 0x01070006u : 0x01050004u;
    const uint32_t vh = __builtin_amdgcn_perm(sc & 0xF0F0F0F0u, 0x64646464u, sel);
    const uint32_t vl = __builtin_amdgcn_perm(sc & 0x0F0F0F0Fu, 0x64646464u, sel);
    return {__builtin_bit_cast(half2v, vh) - (half2v){(_Float16)1152.0f, (_Float16)1152.0f},
            __builtin_bit_cast(half2v, vl) - (half2v){(_Float16)1024.0f, (_Float16)1024.0f}};
}

// The 8 binary16 weights sc * (q6 - 32) of sub-block s (0..3) of a chunk, in MFMA
// A-operand order; ss = stage_scales of the chunk for stage s / 2.  Each is one
// fused multiply-add of the code pair's 256 + c: (256 + c) sc - 288 sc, rounded
// once, i.e. exact while |sc * (q6 - 32)| <= 2048 and within 1/2 ulp otherwise.
// Sub-blocks 0..2 mask their code word; sub-block 3 gathers its code's three bit
// pairs from the other words.
__device__ __forceinline__ half8 decode_frag(const AChunk &c, uint32_t s, _Float16 scf, _Float16 bf)
{
    const half2v sc2 = {scf, scf}, b2 = {bf, bf};
    half2v o[4];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const uint32_t X0 = w ? c.ql.y : c.ql.x, X1 = w ? c.ql.w : c.ql.z, X2 = w ? c.qh.y : c.qh.x;
        const uint32_t M1 = 0x03030303u;
        uint32_t t;
        switch (s) {
        case 0: t = X0 & ~(M1); break;
        case 1: t = X1 & ~(M1); break;
        case 2: t = X2 & ~(M1); break;
        default: t = (((((X2 & M1) << 2) | (X1 & M1)) << 2) | (X0 & M1)) << 2; break;
        }
        o[2 * w] = __builtin_elementwise_fma(codes256(t, false), sc2, b2);
        o[2 * w + 1] = __builtin_elementwise_fma(codes256(t, true), sc2, b2);
    }
    return (half8){o[0][0], o[0][1], o[1][0], o[1][1], o[2][0], o[2][1], o[3][0], o[3][1]};
}
__device__ __forceinline__ half8 decode_frag(const AChunk &c, uint32_t s, const StageScales &ss)
{
    return decode_frag(c, s, ss.sc[s & 1], ss.bias[s & 1]);
}
// The same with the bias formed here (one multiply more per fragment, no
// register held for it across the stage).
__device__ __forceinline__ half8 decode_frag(const AChunk &c, uint32_t s, half2v sc)
{
    return decode_frag(c, s, sc[s & 1], sc[s & 1] * (_Float16)-288.0f);
}

// Q6Tiles -> binary16 fragment copy (kargs.h TILE_H16): workgroup tb (one wave)
// decodes tile-block tb exactly as the GEMMs decode it in registers (same chunk
// loads, same scales, same fused multiply-add per fragment), so the copy holds the
// A fragments those kernels would form, k-step by k-step.
extern "C" __global__ __launch_bounds__(64) void k_q6_tile_h16(const TileH16Args a)
{
    const size_t tb = blockIdx.x, ntb = (size_t)a.src.tiles * a.src.nb;
    const uint32_t lane = threadIdx.x;
    uint8_t *out = a.dst + tb * TILE_H16 + lane * 16;
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) {
        AChunk A[2];
        load_tile_chunks(a.src.base, ntb, tb, h, lane, A);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const half2v s0 = stage_scales(A[0].sc, q).sc, s1 = stage_scales(A[1].sc, q).sc;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) { // k-step ks of stage 2h + q: chunk ks % 2, sub-block 2q + ks / 2
                const half8 f = decode_frag(A[ks & 1], 2 * q + (ks >> 1), (ks & 1) ? s1 : s0);
                *reinterpret_cast<half8 *>(out + ((2 * h + q) * 4 + ks) * 1024) = f;
            }
        }
    }
}

// C[n][row] (+)= sum_k W[row][k] * X[n][k] for weight rows [0, zrows) of group
// z and token columns n < ntok.  Column n reads activation row (tok ? tok[n] :
// n) and writes output row (slot ? slot[n] : n).  The pair form (k_gemm_q6_swiglu)
// multiplies the gate weight w and the up weight w2 by the same activations and
// writes silu(gate) * up (lfm.rs:578-582 SwiGLU, g / (1 + e^-g) * u).
//
// A workgroup computes 256 weight rows x 128 tokens: wave w owns rows 64w..64w+63
// for all 128 tokens (2 x 4 tiles of v_mfma_f32_32x32x16_f16, hi and lo
// activation halves); in the pair form its two row tiles are the same 32 rows of
// the gate and of the up weight (128 rows of each per workgroup), so a lane holds
// a row's gate and up sums side by side.  K advances in 64-wide stages:
//   * weights never touch LDS: each lane loads its rows' Q6_K bytes one half
//     block ahead into registers and decodes the MFMA A fragments itself, the
//     next k-step's fragments while the current k-step's MFMAs run;
//   * activation tiles go global -> LDS directly (buffer_load_dwordx4 ... lds),
//     double-buffered, one barrier per stage;
//   * the super-block scale d is folded into the accumulators: they hold
//     sum_b d_b P_b / u with u the last nonzero d seen, so entering block b
//     multiplies them by u / d_b (blocks with d = 0 contribute zero weights),
//     and the epilogue multiplies by the final u.
// Workgroup i runs on XCD i % 8; tiles are handed out so that each XCD takes a
// contiguous run with the weight rows fastest, and the workgroups resident on
// one XCD share activation tiles in its L2.  With ksplit > 1 the grid's z also
// enumerates K slices: a workgroup runs its slice's blocks only and writes its
// sums to part, which k_gemm_reduce adds up in slice order.
// A lane's 16 accumulator rows of a 32-row tile are rb + 8 (e / 4) + e % 4 (rb =
// the tile's first row + 4 p).  Writes v (add false) or adds it (add true) to those
// rows of out below zrows.  With every row in range the old values are read in one
// batch before the stores: element by element, each read would wait for the
// previous store's address check and read in turn.
__device__ __forceinline__ void store_rows16(float *out, uint32_t rb, uint32_t zrows, const float (&v)[16], bool add)
{
    if (rb + 27 < zrows) {
        float o[16];
        if (add) {
#pragma unroll
            for (int e = 0; e < 16; ++e)
                o[e] = out[rb + 8 * (e / 4) + (e % 4)];
        }
#pragma unroll
        for (int e = 0; e < 16; ++e)
            out[rb + 8 * (e / 4) + (e % 4)] = add ? o[e] + v[e] : v[e];
        return;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t r = rb + 8 * (e / 4) + (e % 4);
        if (r < zrows)
            out[r] = add ? out[r] + v[e] : v[e];
    }
}

// EXACT: the weights are formed with the split scales (stage_scales_split), two
// A fragments per chunk and sub-block, each multiplied by the hi and lo
// activation halves: four matrix-core products per k-step instead of two, and
// exact binary16 weights whatever the scales (the _x kernels).
template <bool PAIR, int NJ, bool EXACT = false>
__device__ __forceinline__ void gemm_body(const GemmArgs &a)
{
    constexpr uint32_t TNW = 32 * NJ; // token columns per workgroup (128, or 32 for small calls)
    // rows of each weight per workgroup; the workgroup's 256 "tile rows" v are
    // rows m0 + v (single) or rows m0 + (v & 127) of weight v >> 7 (pair)
    constexpr uint32_t TMW = PAIR ? TM / 2 : TM;
    uint32_t z, mx, ny;
    {
        const uint32_t gx = gridDim.x, gy = gridDim.y, total = gx * gy * gridDim.z;
        const uint32_t L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
        const uint32_t q = total / 8, r = total % 8, xcd = L % 8, idx = L / 8;
        const uint32_t V = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
        mx = V % gx;
        ny = (V / gx) % gy;
        z = V / (gx * gy);
    }
    // K slice of this workgroup (the whole row unless split)
    const uint32_t nb = a.w.nb, K = nb * 256;
    const uint32_t ks = a.ksplit > 1 ? z / a.nz : 0;
    if (a.ksplit > 1)
        z -= ks * a.nz;
    const uint32_t kb0 = a.ksplit > 1 ? ks * nb / a.ksplit : 0;
    const uint32_t nbl = a.ksplit > 1 ? (ks + 1) * nb / a.ksplit - kb0 : nb;
    const uint32_t m0 = mx * TMW, n0 = ny * TNW;
    const uint32_t ntok = a.counts ? a.counts[z] : a.ntok;
    if (m0 >= a.zrows || n0 >= ntok)
        return;
    const uint32_t *tokl = a.tok ? a.tok + (size_t)z * a.list_stride : nullptr;
    const uint32_t *slotl = a.slot ? a.slot + (size_t)z * a.list_stride : nullptr;
    const __amdgpu_buffer_rsrc_t xh = act_rsrc(a.x_hi), xl = act_rsrc(a.x_lo);
    // the two buffers of the hi and lo tiles as separate arrays, picked by the
    // (unrolled) stage parity: the compiler can then tell that a stage's LDS reads do
    // not touch the buffer the next tile is being loaded into, and does not wait for
    // that load before them
    __shared__ __attribute__((aligned(16))) _Float16 Bh0[TNW * TK], Bh1[TNW * TK];
    __shared__ __attribute__((aligned(16))) _Float16 Bl0[TNW * TK], Bl1[TNW * TK];
    __shared__ float dsh[2][TM], rsh[2][TM];
    // the wave index as a wave-uniform value, so that the row-tile and weight
    // addresses derived from it stay in scalar registers
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t p = lane >> 5, lr = lane & 31;
    const size_t ntb = (size_t)a.w.tiles * nb;
    // row tile i of the wave: tile rows vb[i] .. vb[i] + 31, rows lb[i] .. of weight
    // i (pair), weight tile wt[i] (tiles past the slice's last one read that one:
    // their rows are not stored)
    uint32_t vb[2], lb[2], wt[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        vb[i] = PAIR ? i * 128 + wave * 32 : wave * 64 + i * 32;
        lb[i] = PAIR ? wave * 32 : vb[i];
        wt[i] = z * a.w.gtiles + min((m0 + lb[i]) >> 5, a.w.gtiles - 1);
    }
    // activation pieces: wave w, piece v fills 16-byte units 256v + 64w + lane of
    // a tile, i.e. token t = (tid + 256v) >> 3, unit j = tid & 7, which holds
    // k-piece j ^ ((t >> 1) & 7)
    // (each piece's byte offset, 2 (row * K + its swizzled k-piece), is below the
    // hi / lo buffers' size, which the host keeps under 2^31 bytes)
    uint32_t boff[NJ];
#pragma unroll
    for (int v = 0; v < NJ; ++v) {
        const uint32_t t = (tid + GEMM_NTH * v) >> 3, col = min(n0 + t, ntok - 1);
        boff[v] = ((tokl ? tokl[col] : col) * K + ((tid & 7) ^ ((t >> 1) & 7)) * 8) * 2;
    }
    auto loadA = [=](uint32_t half, AChunk (&A)[2][2]) { // half block of the slice
        const uint32_t kb = kb0 + (half >> 1), h = half & 1;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            load_tile_chunks(PAIR && i ? a.w2.base : a.w.base, ntb, (size_t)wt[i] * nb + kb, h, lane, A[i]);
    };
    auto loadB = [&](uint32_t st, int buf) { // stage st of the slice into buffer buf = st & 1
        _Float16 *bh = buf ? Bh1 : Bh0, *bl = buf ? Bl1 : Bl0;
        static_assert(GEMM_NTH == 256, "piece layout");
        lds_dma_stage<NJ>(xh, xl, boff, (kb0 * 4 + st) * TK * 2, wave, bh, bl);
    };
    // d of tile row tid, block kb of the slice, as binary16 bits (converted where
    // used, so the load does not wait for the weights issued before it)
    auto loadD = [=](uint32_t kb) -> uint32_t {
        const uint8_t *wb = PAIR && tid >= 128 ? a.w2.base : a.w.base;
        const uint32_t v = PAIR ? tid & 127 : tid;
        const uint32_t t = z * a.w.gtiles + min((m0 + v) >> 5, a.w.gtiles - 1);
        return tile_d(wb, ntb, (size_t)t * nb + kb0 + kb, v & 31);
    };
    floatx16 acc[2][NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.f;
    auto rescale = [&](uint32_t rb) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float r = rsh[rb][vb[i] + 8 * (e / 4) + 4 * p + (e % 4)];
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j][e] *= r;
            }
    };
    // thread tid keeps tile row tid's running scale u (TM == GEMM_NTH)
    float u = 1.0f;
    auto set_d = [&](uint32_t slot, float d) {
        dsh[slot][tid] = d;
        const bool nz = d != 0.f;
        rsh[slot][tid] = nz ? u / d : 1.0f;
        u = nz ? d : u;
    };
    const uint32_t nst = nbl * 4, nhb = nbl * 2; // stages; half block hb = stages 2hb, 2hb + 1
    AChunk A[2][2], An[2][2];
    uint32_t dnext = 0;
    float dnextf = 0.f;

    // Stage st = 2 hb + q: issue stage st + 1's tile into buffer 1 - q (every wave
    // finished reading it before the last barrier; stages 0 and 1 come from the
    // prologue), then the next half block's weights and block scale at q = 0, then
    // the MFMAs over buffer q, then wait for stage st + 1's tile and meet at the
    // barrier.  The buffers arrive as restrict-qualified pointers so that the
    // compiler sees that the stage's LDS reads do not touch the tile in flight.
    auto stage = [&](uint32_t hb, int q, const _Float16 *__restrict__ bh, const _Float16 *__restrict__ bl,
                     _Float16 *__restrict__ nh, _Float16 *__restrict__ nl) {
        const uint32_t st = hb * 2 + q;
        if (st >= 1 && st + 1 < nst)
            lds_dma_stage<NJ>(xh, xl, boff, (kb0 * 4 + st + 1) * TK * 2, wave, nh, nl);
        if (q == 0) {
            if (hb > 0) { // the half block's weights, loaded one half block ahead
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int ch = 0; ch < 2; ++ch)
                        A[i][ch] = An[i][ch];
            }
            if (hb + 1 < nhb)
                loadA(hb + 1, An);
            if ((hb & 1) == 0 && hb + 2 < nhb)
                dnext = loadD((hb >> 1) + 1);
        }
        if constexpr (!EXACT) {
        // the stage's scales: sub-blocks 2q, 2q + 1 of each chunk
        half2v ss[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int ch = 0; ch < 2; ++ch)
                ss[i][ch] = stage_scales(A[i][ch].sc, q).sc;
        half8 afc[2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            afc[i] = decode_frag(A[i][0], 2 * q, ss[i][0]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) { // k-step ks: sub-block 2q + ks / 2, chunk ks % 2
            const uint32_t kp = ks * 2 + p;
            // token tile j's fragments are read one tile ahead (two in registers)
            half8 afn[2], bfh[2], bfl[2];
            bfh[0] = lds_frag(bh, swz(lr, kp));
            bfl[0] = lds_frag(bl, swz(lr, kp));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if (j + 1 < NJ) {
                    bfh[(j + 1) & 1] = lds_frag(bh, swz((j + 1) * 32 + lr, kp));
                    bfl[(j + 1) & 1] = lds_frag(bl, swz((j + 1) * 32 + lr, kp));
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afc[i], bfh[j & 1], acc[i][j], 0, 0, 0);
                if (j == 1 && ks < 3) {
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        afn[i] = decode_frag(A[i][(ks + 1) & 1], 2 * q + ((ks + 1) >> 1), ss[i][(ks + 1) & 1]);
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afc[i], bfl[j & 1], acc[i][j], 0, 0, 0);
            }
            if (ks < 3) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    afc[i] = afn[i];
            }
        }
        } else {
        SplitScales sp[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int ch = 0; ch < 2; ++ch)
                sp[i][ch] = stage_scales_split(A[i][ch].sc, q);
        half8 afh[2], afl[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            afh[i] = decode_frag(A[i][0], 2 * q, sp[i][0].sh);
            afl[i] = decode_frag(A[i][0], 2 * q, sp[i][0].sl);
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint32_t kp = ks * 2 + p;
            half8 anh[2], anl[2], bfh[2], bfl[2];
            bfh[0] = lds_frag(bh, swz(lr, kp));
            bfl[0] = lds_frag(bl, swz(lr, kp));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if (j + 1 < NJ) {
                    bfh[(j + 1) & 1] = lds_frag(bh, swz((j + 1) * 32 + lr, kp));
                    bfl[(j + 1) & 1] = lds_frag(bl, swz((j + 1) * 32 + lr, kp));
                }
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afh[i], bfh[j & 1], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bfh[j & 1], acc[i][j], 0, 0, 0);
                }
                if (j == 1 && ks < 3) {
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const SplitScales &n = sp[i][(ks + 1) & 1];
                        anh[i] = decode_frag(A[i][(ks + 1) & 1], 2 * q + ((ks + 1) >> 1), n.sh);
                        anl[i] = decode_frag(A[i][(ks + 1) & 1], 2 * q + ((ks + 1) >> 1), n.sl);
                    }
                }
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afh[i], bfl[j & 1], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bfl[j & 1], acc[i][j], 0, 0, 0);
                }
            }
            if (ks < 3) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    afh[i] = anh[i];
                    afl[i] = anl[i];
                }
            }
        }
        }
        if (q == 0 && (hb & 1) && hb + 1 < nhb) // stage 4kb + 2: publish block kb + 1's scale
            set_d(((hb >> 1) + 1) & 1, dnextf);
        if (st + 1 < nst) {
            // This wave's pieces of stage st + 1 have landed.  At q = 0 the next half
            // block's weights (10 loads) and perhaps a block scale, issued after
            // those pieces (loads retire in issue order), stay in flight: they are
            // used a stage later.  The wait also retires this wave's LDS writes, so a
            // bare barrier (no fence, which would wait for every load) publishes them.
            asm volatile("" ::: "memory");
            if (q == 0 && hb + 1 < nhb) {
                if ((hb & 1) == 0 && hb + 2 < nhb)
                    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(11));
                else
                    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(10));
            } else {
                __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
            }
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
    };
    loadA(0, A);
    loadB(0, 0);
    set_d(0, half_bits_to_float(loadD(0)));
    __builtin_amdgcn_s_waitcnt(0);
    loadB(1, 1);
    __syncthreads();
    for (uint32_t hb = 0; hb < nhb; ++hb) {
        const uint32_t db = (hb >> 1) & 1;
        if ((hb & 1) == 0 && hb > 0)
            rescale(db);
        stage(hb, 0, Bh0, Bl0, Bh1, Bl1);
        stage(hb, 1, Bh1, Bl1, Bh0, Bl0);
        if ((hb & 1) == 0 && hb + 2 < nhb) // landed at the half block's last wait
            dnextf = half_bits_to_float(dnext);
    }
    __syncthreads();
    rsh[0][tid] = u;
    __syncthreads();
    rescale(0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const uint32_t n = n0 + j * 32 + lr;
        if (n >= ntok)
            continue;
        const uint32_t orow = slotl ? slotl[n] : n;
        const float xs = a.xscale[tokl ? tokl[n] : n];
        if (a.ksplit > 1) { // this slice's sums, reduced by k_gemm_reduce
            constexpr uint32_t NW = PAIR ? 2 : 1;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t wi = PAIR ? i : 0;
                float *pp = a.part + ((size_t)(ks * NW + wi) * a.part_rows + orow) * a.zrows;
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    v[e] = acc[i][j][e] * xs;
                store_rows16(pp, m0 + lb[i] + 4 * p, a.zrows, v, false);
            }
            continue;
        }
        float *out = a.c + (size_t)orow * a.ldc + a.col0;
        if (PAIR) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float g = acc[0][j][e] * xs, u = acc[1][j][e] * xs;
                v[e] = g / (1.0f + expf(-g)) * u;
            }
            store_rows16(out, m0 + lb[0] + 4 * p, a.zrows, v, false);
            continue;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e)
                v[e] = acc[i][j][e] * xs;
            store_rows16(out, m0 + lb[i] + 4 * p, a.zrows, v, a.mode != 0);
        }
    }
}

extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_gemm_q6(const GemmArgs a)
{
    gemm_body<false, 4>(a);
}

// 64 token columns per workgroup: for projections whose 128-column grid would leave
// CUs without a second workgroup (few row tiles)
extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_gemm_q6_n64(const GemmArgs a)
{
    gemm_body<false, 2>(a);
}

extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_gemm_q6_swiglu(const GemmArgs a)
{
    gemm_body<true, 4>(a);
}

// Split-scale forms (weights with some |sc| > 64): 64 token columns per workgroup,
// so that the second set of weight fragments fits the registers.
extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_gemm_q6_x(const GemmArgs a)
{
    gemm_body<false, 2, true>(a);
}

extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_gemm_q6_swiglu_x(const GemmArgs a)
{
    gemm_body<true, 2, true>(a);
}

// The large-call GEMM over the binary16 fragment copy (Q6Tiles::h16, made once at
// finalize by k_q6_tile_h16): gemm_body's workgroup tiles, activation staging,
// block-scale folding and epilogue, but each wave loads its A fragments ready-made,
// one 16-byte load per lane, fragment and k-step (1 KB contiguous per wave),
// instead of loading Q6_K bytes and decoding them: the k-loop is loads, LDS
// fragment reads and MFMAs.  The products are those of gemm_body (the
// copy holds the fragments its decode forms).  Large calls only: one K slice.
template <bool PAIR, int NJ>
__device__ __forceinline__ void gemm_body_h(const GemmArgs &a)
{
    constexpr uint32_t TNW = 32 * NJ;
    constexpr uint32_t TMW = PAIR ? TM / 2 : TM;
    uint32_t z, mx, ny;
    {
        const uint32_t gx = gridDim.x, gy = gridDim.y, total = gx * gy * gridDim.z;
        const uint32_t L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
        const uint32_t q = total / 8, r = total % 8, xcd = L % 8, idx = L / 8;
        const uint32_t V = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
        // Within a weight slice, groups of 8 token tiles with the row tiles next: the
        // workgroups resident on one XCD (a run of consecutive V) then cover about 8
        // row tiles x 8 token tiles, whose weights and activations its L2 shares.
        // (Row tiles fastest over all token tiles, as gemm_body orders them, reads
        // the whole weight once per token tile: 2.4 times the Q6_K bytes here.)
        const uint32_t per = gx * gy, Vz = V % per, g = Vz / (gx * 8), w = Vz - g * gx * 8;
        const uint32_t ng = min(8u, gy - g * 8);
        mx = gx > 8 ? w / ng : Vz % gx;
        ny = gx > 8 ? g * 8 + w % ng : Vz / gx;
        z = V / per;
    }
    const uint32_t nb = a.w.nb, K = nb * 256;
    const uint32_t m0 = mx * TMW, n0 = ny * TNW;
    const uint32_t ntok = a.counts ? a.counts[z] : a.ntok;
    if (m0 >= a.zrows || n0 >= ntok)
        return;
    const uint32_t *tokl = a.tok ? a.tok + (size_t)z * a.list_stride : nullptr;
    const uint32_t *slotl = a.slot ? a.slot + (size_t)z * a.list_stride : nullptr;
    const __amdgpu_buffer_rsrc_t xh = act_rsrc(a.x_hi), xl = act_rsrc(a.x_lo);
    __shared__ __attribute__((aligned(16))) _Float16 Bh0[TNW * TK], Bh1[TNW * TK];
    __shared__ __attribute__((aligned(16))) _Float16 Bl0[TNW * TK], Bl1[TNW * TK];
    __shared__ float dsh[2][TM], rsh[2][TM];
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t p = lane >> 5, lr = lane & 31;
    const size_t ntb = (size_t)a.w.tiles * nb;
    uint32_t vb[2], lb[2];
    const uint8_t *hw[2]; // row tile i's fragments: tile-blocks wt * nb .. are consecutive
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        vb[i] = PAIR ? i * 128 + wave * 32 : wave * 64 + i * 32;
        lb[i] = PAIR ? wave * 32 : vb[i];
        const uint32_t wt = z * a.w.gtiles + min((m0 + lb[i]) >> 5, a.w.gtiles - 1);
        hw[i] = (PAIR && i ? a.w2.h16 : a.w.h16) + (size_t)wt * nb * TILE_H16 + lane * 16;
    }
    uint32_t boff[NJ];
#pragma unroll
    for (int v = 0; v < NJ; ++v) {
        const uint32_t t = (tid + GEMM_NTH * v) >> 3, col = min(n0 + t, ntok - 1);
        boff[v] = ((tokl ? tokl[col] : col) * K + ((tid & 7) ^ ((t >> 1) & 7)) * 8) * 2;
    }
    // stage st's fragments of k-step ks (block st / 4, k-step 4 (st % 4) + ks of it)
    auto loadF = [&](uint32_t st, int ks, half8 (&F)[2][4]) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            F[i][ks] = *reinterpret_cast<const half8 *>(hw[i] + (size_t)st * 4096 + ks * 1024);
    };
    auto loadD = [=](uint32_t kb) -> uint32_t {
        const uint8_t *wb = PAIR && tid >= 128 ? a.w2.base : a.w.base;
        const uint32_t v = PAIR ? tid & 127 : tid;
        const uint32_t t = z * a.w.gtiles + min((m0 + v) >> 5, a.w.gtiles - 1);
        return tile_d(wb, ntb, (size_t)t * nb + kb, v & 31);
    };
    floatx16 acc[2][NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.f;
    auto rescale = [&](uint32_t rb) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float r = rsh[rb][vb[i] + 8 * (e / 4) + 4 * p + (e % 4)];
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j][e] *= r;
            }
    };
    float u = 1.0f;
    auto set_d = [&](uint32_t slot, float d) {
        dsh[slot][tid] = d;
        const bool nz = d != 0.f;
        rsh[slot][tid] = nz ? u / d : 1.0f;
        u = nz ? d : u;
    };
    const uint32_t nst = nb * 4;
    uint32_t dnext = 0;
    float dnextf = 0.f;

    // Stage st = 4 kb + sb over tile buffer sb % 2 and the fragments F: issue stage
    // st + 1's tile into the other buffer (and at sb = 0 block kb + 1's scale), then
    // the k-steps, each followed by the load of stage st + 1's fragments of that
    // k-step into the registers it just used (one register set: in isolated runs 5-9 %
    // faster than a second set for two stages ahead, the same in the whole prompt,
    // with 24 fewer VGPRs; loads issued together at the stage start were slower
    // still), then wait for stage st + 1's tile (the 8 fragment loads
    // issued after it stay in flight: loads retire in issue order) and meet at the
    // barrier.
    auto stage = [&](uint32_t st, const _Float16 *__restrict__ bh, const _Float16 *__restrict__ bl,
                     _Float16 *__restrict__ nh, _Float16 *__restrict__ nl, half8 (&F)[2][4]) {
        const uint32_t kb = st >> 2, sb = st & 3;
        // Every load is issued without a branch around it (past the last stage and
        // block, the last ones again, unused): a load under a branch leaves the
        // compiler's wait counts unknown at the join, after which the first use of
        // a fragment would wait for every load issued after it.
        const uint32_t sn = min(st + 1, nst - 1);
        if (sb == 0 && kb > 0)
            rescale(kb & 1);
        issue_fence();
        lds_dma_stage<NJ>(xh, xl, boff, sn * TK * 2, wave, nh, nl);
        issue_fence();
        if (sb == 0)
            dnext = loadD(min(kb + 1, nb - 1));
        issue_fence();
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint32_t kp = ks * 2 + p;
            half8 bfh[2], bfl[2];
            bfh[0] = lds_frag(bh, swz(lr, kp));
            bfl[0] = lds_frag(bl, swz(lr, kp));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if (j + 1 < NJ) {
                    bfh[(j + 1) & 1] = lds_frag(bh, swz((j + 1) * 32 + lr, kp));
                    bfl[(j + 1) & 1] = lds_frag(bl, swz((j + 1) * 32 + lr, kp));
                }
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[i][ks], bfh[j & 1], acc[i][j], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(F[i][ks], bfl[j & 1], acc[i][j], 0, 0, 0);
            }
            issue_fence();
            loadF(sn, ks, F);
            issue_fence();
        }
        if (sb == 2 && kb + 1 < nb) // publish block kb + 1's scale (landed by stage 4 kb + 1's wait)
            set_d((kb + 1) & 1, dnextf);
        // stage st + 1's tile has landed (this wave's pieces; the wait also retires
        // its LDS reads and writes and the scale issued after the tile); stage st +
        // 1's fragments stay in flight, and the barrier publishes the tile
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(8));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (sb == 1)
            dnextf = half_bits_to_float(dnext);
    };
    half8 F[2][4];
    lds_dma_stage<NJ>(xh, xl, boff, 0, wave, Bh0, Bl0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
        loadF(0, ks, F);
    set_d(0, half_bits_to_float(loadD(0)));
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (uint32_t kb = 0; kb < nb; ++kb) {
        stage(4 * kb + 0, Bh0, Bl0, Bh1, Bl1, F);
        stage(4 * kb + 1, Bh1, Bl1, Bh0, Bl0, F);
        stage(4 * kb + 2, Bh0, Bl0, Bh1, Bl1, F);
        stage(4 * kb + 3, Bh1, Bl1, Bh0, Bl0, F);
    }
    __syncthreads();
    rsh[0][tid] = u;
    __syncthreads();
    rescale(0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const uint32_t n = n0 + j * 32 + lr;
        if (n >= ntok)
            continue;
        const uint32_t orow = slotl ? slotl[n] : n;
        const float xs = a.xscale[tokl ? tokl[n] : n];
        float *out = a.c + (size_t)orow * a.ldc + a.col0;
        if (PAIR) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float g = acc[0][j][e] * xs, uu = acc[1][j][e] * xs;
                v[e] = g / (1.0f + expf(-g)) * uu;
            }
            store_rows16(out, m0 + lb[0] + 4 * p, a.zrows, v, false);
            continue;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e)
                v[e] = acc[i][j][e] * xs;
            store_rows16(out, m0 + lb[i] + 4 * p, a.zrows, v, a.mode != 0);
        }
    }
}

extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_gemm_h16(const GemmArgs a)
{
    gemm_body_h<false, 4>(a);
}

// (152 VGPRs: three waves per SIMD)
extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(3, 3))) void
k_gemm_h16_n64(const GemmArgs a)
{
    gemm_body_h<false, 2>(a);
}

extern "C" __global__ __launch_bounds__(GEMM_NTH) __attribute__((amdgpu_waves_per_eu(2, 2))) void
k_gemm_swiglu_h16(const GemmArgs a)
{
    gemm_body_h<true, 4>(a);
}

// The same products for calls of up to 128 tokens (chunked prefill: about 8
// tokens per expert at 64 tokens), 32 tokens per workgroup: a quarter of the
// padded matrix-core work, and every wave runs on its own.  A lane loads its
// weight rows' Q6_K bytes a half block ahead and its token column's activation
// fragments (hi, lo) a stage ahead straight into registers; the block scales
// are exchanged between lanes by shuffles (lane l holds row l's running scale),
// so there is no LDS tile and no barrier, and each wave waits only for the
// loads its next instructions use.  Same arithmetic per (row, token) as
// gemm_body.  NI: 32-row tiles per wave (the pair form: its gate and up tile).
// EXACT: split-scale weights as in gemm_body (the _x kernels).
template <bool PAIR, int NI, int G, bool EXACT = false>
__device__ __forceinline__ void gemm_small_body(const GemmArgs &a)
{
    static_assert(!PAIR || NI == 2, "the pair form holds a gate and an up tile per wave");
    constexpr uint32_t TMW = PAIR ? TM / 2 : 128 * NI; // rows of each weight per workgroup
    uint32_t z, mx, ny;
    {
        const uint32_t gx = gridDim.x, gy = gridDim.y, total = gx * gy * gridDim.z;
        const uint32_t L = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
        const uint32_t q = total / 8, r = total % 8, xcd = L % 8, idx = L / 8;
        const uint32_t V = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
        mx = V % gx;
        ny = (V / gx) % gy;
        z = V / (gx * gy);
    }
    const uint32_t nb = a.w.nb, K = nb * 256;
    const uint32_t ks = a.ksplit > 1 ? z / a.nz : 0;
    if (a.ksplit > 1)
        z -= ks * a.nz;
    const uint32_t kb0 = a.ksplit > 1 ? ks * nb / a.ksplit : 0;
    const uint32_t nbl = a.ksplit > 1 ? (ks + 1) * nb / a.ksplit - kb0 : nb;
    const uint32_t m0 = mx * TMW, n0 = ny * 32;
    const uint32_t ntok = a.counts ? a.counts[z] : a.ntok;
    if (m0 >= a.zrows || n0 >= ntok)
        return;
    const uint32_t *tokl = a.tok ? a.tok + (size_t)z * a.list_stride : nullptr;
    const uint32_t *slotl = a.slot ? a.slot + (size_t)z * a.list_stride : nullptr;
    const __amdgpu_buffer_rsrc_t xh = act_rsrc(a.x_hi), xl = act_rsrc(a.x_lo);
    // the wave index as a wave-uniform value, so that the row-tile and weight
    // addresses derived from it stay in scalar registers
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t p = lane >> 5, lr = lane & 31;
    const size_t ntb = (size_t)a.w.tiles * nb;
    // row tile i of the wave: rows lb[i] .. + 31 of the workgroup's, weight tile wt[i]
    // (tiles past the slice's last one read that one: their rows are not stored)
    uint32_t lb[NI], wt[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        lb[i] = PAIR ? wave * 32 : wave * 32 * NI + i * 32;
        wt[i] = z * a.w.gtiles + min((m0 + lb[i]) >> 5, a.w.gtiles - 1);
    }
    // Activations token-blocked: the workgroup's 32 columns are logical tile lt
    // (group z's tiles start at z * rpz / 32), whose 64-wide stage is 4 KB of hi and
    // 4 KB of lo, contiguous.  The four waves load a stage into one LDS buffer
    // (wave w: k-pieces 2w, 2w + 1, i.e. kilobyte w of each half; lanes past the
    // tile's last column re-read that column, so an expert tile of ~8 tokens reads
    // ~8 rows' bytes) and read their MFMA B fragments from there.  Byte offsets stay
    // below 2^31 (the host bounds the activation copies).
    const uint32_t lt = (tokl ? z * (a.rpz >> 5) : 0u) + ny;
    const uint32_t bsrc = 2 * (lt * (K >> 3) * 256 + (2 * wave + p) * 256 + min(lr, ntok - 1 - n0) * 8);
    // this lane's token column's activation scales: logical row lrow, half-blocks of K
    const float *bsc = a.bscale + (size_t)(lt * 32 + min(lr, ntok - 1 - n0)) * (K >> 7);
    // G + 4 stage buffers of 8 KB, hi then lo (stage s in buffer s % (G + 4));
    // every LDS read of them is in assembly, so the compiler adds no waits for the
    // tiles in flight and the buffer can be picked at run time
    static_assert(G == 2 || G == 4, "a barrier every 2 or 4 stages");
    constexpr uint32_t NBUF = G + 4;
    __shared__ __attribute__((aligned(16))) _Float16 Bs[NBUF][2 * 8 * 256];
    typedef AChunk BlockW[2][NI][2]; // a block's weights: [half][row tile][chunk]
    auto loadA = [=](uint32_t half, AChunk (&A)[NI][2]) {
        const uint32_t kb = kb0 + (half >> 1), h = half & 1;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            load_tile_chunks<true>(PAIR && i ? a.w2.base : a.w.base, ntb, (size_t)wt[i] * nb + kb, h, lane, A[i]);
    };
    // stage st's tile into its buffer (this wave's two 16-byte pieces per lane)
    auto loadB = [&](uint32_t st) {
        const uint32_t o = bsrc + (kb0 * 4 + st) * TK * 32 * 2;
        _Float16 *dst = Bs[st % NBUF];
        lds_dma16(xh, o, &dst[wave * 512]);
        lds_dma16(xl, o, &dst[8 * 256 + wave * 512]);
    };
    // this lane's A rows' block scales d, block kb of the slice, as binary16 bits
    // (converted where used, so the load does not wait for the weights issued before it)
    // and the activation scales of its half-blocks (two loads more)
    auto loadD = [=](uint32_t kb, uint32_t (&d)[NI], float (&ts)[2]) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
            d[i] = tile_d(PAIR && i ? a.w2.base : a.w.base, ntb, (size_t)wt[i] * nb + kb0 + kb, lr);
        ts[0] = bsc[2 * (kb0 + kb)];
        ts[1] = bsc[2 * (kb0 + kb) + 1];
    };
    floatx16 acc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            acc[i][e] = 0.f;
    // accumulator element e of a lane is row 8 (e / 4) + 4p + e % 4 of its tile,
    // whose factor v lives in lane (that row) % 32: the wave passes the 32 factors
    // through its own LDS slots (one store, four 16-byte reads of 4 rows each,
    // in order within the wave) instead of 16 lane shuffles
    // (in assembly: the compiler would wait for the activation tiles in flight
    // before reading an LDS array it cannot tell apart from their buffers)
    __shared__ __attribute__((aligned(16))) float rowf[4][NI][32];
    // (times c, this lane's own factor: its token column's activation-scale ratio)
    auto by_row = [&](int i, float v, float c) {
        floatx4 f[4]; // lanes lr and lr + 32 store the same value
        lds_rowf(lds_addr(&rowf[wave][i][lr]), v, lds_addr(&rowf[wave][i][4 * p]), f);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][4 * k + j] *= f[k][j] * c;
    };
    float u[NI], dcur[NI];
    uint32_t dnext[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
        u[i] = 1.0f, dnext[i] = 0;
    // The activations of half-block h of this lane's column were stored divided by
    // s_h: the accumulators hold sum_h s_h P_h / ut, multiplied by ut / s_h when
    // half-block h starts (powers of two: exact) and by the final ut at the end.
    float ut = 1.0f, tnext[2] = {1.0f, 1.0f}, tcur1 = 1.0f;
    auto enter_block = [&](bool first) { // accumulators: sum_b d_b P_b / u
        const float c = ut / tnext[0];
        ut = tnext[0];
        tcur1 = tnext[1];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const bool nz = dcur[i] != 0.f;
            const float r = nz ? u[i] / dcur[i] : 1.0f;
            u[i] = nz ? dcur[i] : u[i];
            if (!first)
                by_row(i, r, c);
        }
    };
    auto enter_half = [&]() { // the block's second half-block
        const float c = ut / tcur1;
        ut = tcur1;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][e] *= c;
    };
    const uint32_t nst = nbl * 4;

    // Stage s = 4 kb + j.  The workgroup meets at a barrier after every G-th stage
    // only: the first stage of a group issues the tiles of stages s + 4 .. s + 3 + G
    // into buffers whose stages every wave left before the last barrier.  Then the
    // next block's first half of the weights with its scales, and later its second
    // half (see below).  Loads retire in issue order, so each wait for the tiles and
    // weights of the coming stages leaves everything issued after them in flight:
    // the weights have two (G = 4) or three stages to arrive, the tiles at least four.
    auto stage = [&](uint32_t kb, int j, BlockW &W, BlockW &N) {
        const uint32_t st = kb * 4 + j;
        const bool more = kb + 1 < nbl; // a next block exists
        if (j == 0) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
                dcur[i] = half_bits_to_float(dnext[i]);
            enter_block(kb == 0);
        }
        if (j == 2)
            enter_half();
        issue_fence();
        if (j % G == 0) {
#pragma unroll
            for (int u = 0; u < G; ++u)
                if (st + 4 + u < nst)
                    loadB(st + 4 + u);
        }
        issue_fence();
        // the next block's halves of the weights: G = 2 at j = 0 (with the scales)
        // and 2; G = 4 a stage later, at j = 1 and 3 (measured faster: 188 vs 193 ms
        // for a 3840-token prompt in 64-token calls)
        constexpr int JA = G == 4 ? 1 : 0, JB = JA + 2;
        if ((j == JA || j == JB) && more) {
            loadA(2 * (kb + 1) + (j == JB), N[j == JB]);
            if (j == JA)
                loadD(kb + 1, dnext, tnext);
        }
        issue_fence();
        const int q = j & 1;
        AChunk (&A)[NI][2] = W[j >> 1];
        half8 bch[4], bcl[4];
        // k-step kq reads k-piece 2 kq + p of row lr
        lds_frags_issue(lds_addr(Bs[st % NBUF]) + (p * 256 + lr * 8) * 2, bch, bcl);
        if constexpr (!EXACT) {
        half8 afc[NI];
        // the stage's scales: sub-blocks 2q, 2q + 1 of each chunk
        StageScales ss[NI][2];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int ch = 0; ch < 2; ++ch)
                ss[i][ch] = stage_scales(A[i][ch].sc, q);
#pragma unroll
        for (int i = 0; i < NI; ++i)
            afc[i] = decode_frag(A[i][0], 2 * q, ss[i][0]);
        lds_frags_wait(bch, bcl);
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) {
            half8 afn[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afc[i], bch[kq], acc[i], 0, 0, 0);
            if (kq < 3) {
#pragma unroll
                for (int i = 0; i < NI; ++i)
                    afn[i] = decode_frag(A[i][(kq + 1) & 1], 2 * q + ((kq + 1) >> 1), ss[i][(kq + 1) & 1]);
            }
#pragma unroll
            for (int i = 0; i < NI; ++i)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afc[i], bcl[kq], acc[i], 0, 0, 0);
            if (kq < 3) {
#pragma unroll
                for (int i = 0; i < NI; ++i)
                    afc[i] = afn[i];
            }
        }
        } else {
        half8 afh[NI], afl[NI];
        SplitScales sp[NI][2];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int ch = 0; ch < 2; ++ch)
                sp[i][ch] = stage_scales_split(A[i][ch].sc, q);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            afh[i] = decode_frag(A[i][0], 2 * q, sp[i][0].sh);
            afl[i] = decode_frag(A[i][0], 2 * q, sp[i][0].sl);
        }
        lds_frags_wait(bch, bcl);
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) {
            half8 anh[NI], anl[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afh[i], bch[kq], acc[i], 0, 0, 0);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bch[kq], acc[i], 0, 0, 0);
            }
            if (kq < 3) {
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const SplitScales &n = sp[i][(kq + 1) & 1];
                    anh[i] = decode_frag(A[i][(kq + 1) & 1], 2 * q + ((kq + 1) >> 1), n.sh);
                    anl[i] = decode_frag(A[i][(kq + 1) & 1], 2 * q + ((kq + 1) >> 1), n.sl);
                }
            }
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afh[i], bcl[kq], acc[i], 0, 0, 0);
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afl[i], bcl[kq], acc[i], 0, 0, 0);
            }
            if (kq < 3) {
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    afh[i] = anh[i];
                    afl[i] = anl[i];
                }
            }
        }
        }
        if (G == 2 && (j & 1) && st + 1 < nst) {
            // Stages st + 1 and st + 2 have their tiles and weights, and every wave is
            // done with buffers st - 1 and st.  Still in flight (issued after what is
            // waited for): j = 1: the tiles of stage st - 1 (4 loads) and the next
            // block's first half + scales (6 NI) issued there; j = 3: the tiles of
            // stage st - 1 and the next block's second half (5 NI).  Without a next
            // block nothing was issued at stage st - 1, and the last stages wait for
            // all.
            asm volatile("" ::: "memory");
            if (j == 1) {
                if (more)
                    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(4 + 6 * NI + 2));
                else
                    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
            } else {
                __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(4 + 5 * NI)); // j = 3 ends a block that has a next
            }
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        if (G == 4 && j == 1 && st + 1 < nst) {
            // the block's second half of the weights has landed (no barrier: the
            // tiles of stages st + 1, st + 2 came with the last one); in flight: the
            // 4 tiles of stage st - 1 (8 loads) and the next block's first half +
            // scales of this stage (6 NI)
            asm volatile("" ::: "memory");
            if (more)
                __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(8 + 6 * NI + 2));
            else
                __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(0));
            asm volatile("" ::: "memory");
        }
        if (G == 4 && j == 3 && st + 1 < nst) {
            // the next block's tiles, first half of the weights and scales have
            // landed and every wave is done with this block's buffers; in flight: the
            // next block's second half (5 NI)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0(5 * NI));
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
    };
    auto block = [&](uint32_t kb, BlockW &W, BlockW &N) {
        stage(kb, 0, W, N);
        stage(kb, 1, W, N);
        stage(kb, 2, W, N);
        stage(kb, 3, W, N);
    };
    // Prologue: what stages -4 .. -1 of a block before the first would have issued
    // (G = 2: tiles 0, 1 and the first half block of weights with the scales at -4,
    // tiles 2, 3 and the second half at -2; G = 4: tiles 0 .. 3, the first half and
    // the scales at -4, the second half at -2), then the wait and barrier of stage -1.
    BlockW S0, S1;
    loadB(0);
    loadB(1);
    if (G == 4) {
        loadB(2);
        loadB(3);
    }
    issue_fence();
    loadA(0, S0[0]);
    loadD(0, dnext, tnext);
    issue_fence();
    if (G == 2) {
        loadB(2);
        loadB(3);
    }
    issue_fence();
    loadA(1, S0[1]);
    issue_fence();
    __builtin_amdgcn_s_waitcnt(WAITCNT_VM_LGKM0((G == 2 ? 4 : 0) + 5 * NI));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    uint32_t kb = 0;
    for (; kb + 1 < nbl; kb += 2) {
        block(kb, S0, S1);
        block(kb + 1, S1, S0);
    }
    if (kb < nbl)
        block(kb, S0, S1);
#pragma unroll
    for (int i = 0; i < NI; ++i)
        by_row(i, u[i], 1.0f);
    const float xs = ut;
    if (PAIR && a.y_hi) { // uniform (ksplit 1): the SwiGLU output goes out split
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float g = acc[0][e] * xs, uu = acc[NI - 1][e] * xs;
            v[e] = g / (1.0f + expf(-g)) * uu;
        }
        // the largest magnitude of this column's 128 rows: 16 per lane, both lane
        // halves, the four waves (lanes past the last column hold its copies)
        float m = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e)
            m = fmaxf(m, fabsf(v[e]));
        const float2v mh = wave_halves(m);
        m = fmaxf(mh[0], mh[1]);
        __shared__ float cmax[4][32];
        if (p == 0)
            cmax[wave][lr] = m;
        __syncthreads();
        m = fmaxf(fmaxf(cmax[0][lr], cmax[1][lr]), fmaxf(cmax[2][lr], cmax[3][lr]));
        int ex = 0;
        if (m > 0.f && m <= 3.0e38f)
            frexpf(m, &ex);
        const float sc = m > 0.f ? ldexpf(1.0f, ex - 14) : 1.0f, rs = 1.0f / sc;
        const uint32_t n = n0 + lr;
        if (n >= ntok)
            return;
        const uint32_t L = (tokl ? z * a.rpz : 0u) + n, Ko = a.zrows;
        if (wave == 0 && p == 0)
            a.y_bscale[(size_t)L * (Ko >> 7) + (m0 >> 7)] = sc;
        // element e is row m0 + 32 wave + 8 (e / 4) + 4 p + e % 4: per e / 4, four
        // consecutive k of one 8-wide piece, the lane half p's four halves of it
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            half4v h, l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 hh, ll;
                split_f16(v[4 * q + e] * rs, hh, ll);
                h[e] = hh;
                l[e] = ll;
            }
            const size_t o = blocked_index(L, m0 + lb[0] + 8 * q + 4 * p, Ko);
            *reinterpret_cast<half4v *>(a.y_hi + o) = h;
            *reinterpret_cast<half4v *>(a.y_lo + o) = l;
        }
        return;
    }
    const uint32_t n = n0 + lr;
    if (n >= ntok)
        return;
    const uint32_t orow = slotl ? slotl[n] : n;
    if (a.ksplit > 1) {
        constexpr uint32_t NW = PAIR ? 2 : 1;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            float *pp = a.part + ((size_t)(ks * NW + (PAIR ? i : 0)) * a.part_rows + orow) * a.zrows;
            float v[16];
#pragma unroll
            for (int e = 0; e < 16; ++e)
                v[e] = acc[i][e] * xs;
            store_rows16(pp, m0 + lb[i] + 4 * p, a.zrows, v, false);
        }
        return;
    }
    float *out = a.c + (size_t)orow * a.ldc + a.col0;
    if (PAIR) {
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float g = acc[0][e] * xs, uu = acc[NI - 1][e] * xs;
            v[e] = g / (1.0f + expf(-g)) * uu;
        }
        store_rows16(out, m0 + lb[0] + 4 * p, a.zrows, v, false);
        return;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        float v[16];
#pragma unroll
        for (int e = 0; e < 16; ++e)
            v[e] = acc[i][e] * xs;
        store_rows16(out, m0 + lb[i] + 4 * p, a.zrows, v, a.mode != 0);
    }
}

// Two 32-row tiles per wave (two workgroups per CU): a barrier once per block.
extern "C" __global__ __launch_bounds__(GEMM_NTH) void k_gemm_q6_t32(const GemmArgs a)
{
    gemm_small_body<false, 2, 4>(a);
}

extern "C" __global__ __launch_bounds__(GEMM_NTH) void k_gemm_q6_swiglu_t32(const GemmArgs a)
{
    gemm_small_body<true, 2, 4>(a);
}

// One 32-row tile per wave (128 rows per workgroup, 144 VGPRs: three waves per
// SIMD): faster for the ungrouped projections of up to 2048 rows at 64 tokens,
// slower for the expert and 6144-row shapes.
extern "C" __global__ __launch_bounds__(GEMM_NTH) void k_gemm_q6_t32n1(const GemmArgs a)
{
    gemm_small_body<false, 1, 2>(a); // three workgroups per CU: 6 tile buffers fit their LDS
}

// Split-scale forms (weights with some |sc| > 64): one 32-row tile per wave for
// single weights, the gate and up tiles for the pair.
extern "C" __global__ __launch_bounds__(GEMM_NTH) void k_gemm_q6_t32x(const GemmArgs a)
{
    gemm_small_body<false, 1, 2, true>(a);
}

extern "C" __global__ __launch_bounds__(GEMM_NTH) void k_gemm_q6_swiglu_t32x(const GemmArgs a)
{
    gemm_small_body<true, 2, 4, true>(a);
}

// Sums the K slices of a split GEMM in slice order and applies its epilogue:
// c = v, c += v (mode 1), or silu(g) * u for the pair form.  One thread per
// output element (row blockIdx.x * 256 + tid of output row blockIdx.y).
// Router partials of the rows a reduce workgroup just finished (GemmReduceArgs):
// thread (part = tid / 64, expert e = tid % 64) dots the 64 rows of its part with
// router row e; the four parts are added in order.  The router rows are loaded
// before the slices are summed.
struct RouterRows {
    float4 w[16];
    float nw; // rnorm of this thread's row
};
__device__ __forceinline__ RouterRows router_rows_load(const GemmReduceArgs &a)
{
    RouterRows rr;
    const uint32_t tid = threadIdx.x, e = min(tid & 63, a.n_expert - 1), part = tid >> 6;
    const float4 *w = reinterpret_cast<const float4 *>(a.rw + (size_t)e * a.zrows + blockIdx.x * 256 + part * 64);
#pragma unroll
    for (int i = 0; i < 16; ++i)
        rr.w[i] = w[i];
    rr.nw = a.rnorm[blockIdx.x * 256 + tid];
    return rr;
}
__device__ __forceinline__ void router_partials(const GemmReduceArgs &a, const RouterRows &rr, float xn)
{
    __shared__ __attribute__((aligned(16))) float xw[256];
    __shared__ float red[4][64], ssw[4];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, t = blockIdx.y;
    xw[tid] = xn * rr.nw;
    const float ss = wave_sum(xn * xn);
    if (lane == 0)
        ssw[wave] = ss;
    __syncthreads();
    const float4 *xv = reinterpret_cast<const float4 *>(xw + wave * 64);
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 x4 = xv[i];
        dot = fmaf(x4.x, rr.w[i].x, dot);
        dot = fmaf(x4.y, rr.w[i].y, dot);
        dot = fmaf(x4.z, rr.w[i].z, dot);
        dot = fmaf(x4.w, rr.w[i].w, dot);
    }
    red[wave][lane] = dot;
    __syncthreads();
    const size_t blk = (size_t)t * gridDim.x + blockIdx.x;
    if (tid < a.n_expert)
        a.rpart[blk * a.n_expert + tid] = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
    if (tid == 64)
        a.rss[blk] = ((ssw[0] + ssw[1]) + ssw[2]) + ssw[3];
}

extern "C" __global__ __launch_bounds__(WG_THREADS) void k_gemm_reduce(const GemmReduceArgs a)
{
    const uint32_t r = blockIdx.x * WG_THREADS + threadIdx.x, orow = blockIdx.y;
    if (a.rw) { // uniform; every row is in range (zrows is a multiple of 256)
        const RouterRows rr = router_rows_load(a);
        const size_t slice = (size_t)a.part_rows * a.zrows, at = (size_t)orow * a.zrows + r;
        float *out = a.c + (size_t)orow * a.ldc + a.col0 + r;
        const float old = *out;
        float v[1] = {0.f};
        slice_sums<1>(a.part + at, slice, a.ksplit, {0}, v);
        const float xn = a.mode ? old + v[0] : v[0];
        *out = xn;
        if (a.counts && blockIdx.x == 0 && orow == 0 && threadIdx.x < a.n_expert)
            a.counts[threadIdx.x] = 0;
        router_partials(a, rr, xn);
        return;
    }
    if (r >= a.zrows || (a.n_used && orow % 4 >= a.n_used))
        return;
    const size_t slice = (size_t)a.part_rows * a.zrows, at = (size_t)orow * a.zrows + r;
    float *out = a.c + (size_t)orow * a.ldc + a.col0 + r;
    if (a.pair) { // slice s holds the gate sums at 2s, the up sums at 2s + 1
        float gu[2] = {0.f, 0.f};
        slice_sums<2>(a.part + at, 2 * slice, a.ksplit, {0, slice}, gu);
        const float g = gu[0], u = gu[1];
        *out = g / (1.0f + expf(-g)) * u;
        return;
    }
    const float old = *out; // issued with the slices (unused unless accumulating)
    float v[1] = {0.f};
    slice_sums<1>(a.part + at, slice, a.ksplit, {0}, v);
    *out = a.mode ? old + v[0] : v[0];
}
// ------------------------------------------------------------------ short conv
// The LFM2 short conv keeps only the previous two values of bx = B*X, so each
// (t, ch) output depends on inputs t-2, t-1, t only: the T tokens of a chunk are
// computed in parallel with the reference's per-element operation order
// (lfm.rs:464-533: co = ((0 + s0*w0) + s1*w1) + bx*w2, y = C*co, no contraction).
// With a split-K in_proj the kernel adds its partial sums itself (each B and X
// value is read by the three tokens that use it), in slice order as
// k_gemm_reduce would.  The new state (bx[T-2], bx[T-1]), or (s1, bx[0]) for T = 1,
// goes to state_next: workgroups of the first tokens may still read the old one.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_conv_prefill(const ConvPrefillArgs a)
{
#pragma clang fp contract(off)
    const uint32_t ch = blockIdx.x * WG_THREADS + threadIdx.x;
    const uint32_t t = blockIdx.y;
    if (ch >= a.dim || t >= a.T)
        return;
    const size_t D3 = 3 * (size_t)a.dim, slice = (size_t)a.T * D3;
    // B and X of tokens t-2, t-1, t (clamped to token 0: values for t < 2 come from
    // the state), C of token t, all slices' loads issued together
    const uint32_t t2 = t >= 2 ? t - 2 : 0, t1 = t >= 1 ? t - 1 : 0;
    float v[7];
    const size_t base = ch;
    slice_sums<7>(a.bcx + base, slice, a.ksplit,
                  {t2 * D3, t2 * D3 + 2 * a.dim, t1 * D3, t1 * D3 + 2 * a.dim, t * D3, t * D3 + 2 * a.dim,
                   t * D3 + a.dim},
                  v);
    float st0 = 0.f, st1 = 0.f;
    if (t < 2) { // uniform
        st0 = a.state[ch * 2];
        st1 = a.state[ch * 2 + 1];
    }
    const float bx = v[4] * v[5];
    const float s0 = t >= 2 ? v[0] * v[1] : t == 1 ? st1 : st0;
    const float s1 = t >= 1 ? v[2] * v[3] : st1;
    const float *w3 = a.conv_w + ch * 3;
    float co = 0.0f;
    co = co + s0 * w3[0];
    co = co + s1 * w3[1];
    co = co + bx * w3[2];
    const float yv = v[6] * co;
    if (a.y_hi) { // uniform
        // the largest magnitude of this half-block's 128 channels (waves 2h, 2h + 1)
        __shared__ float hmax[4];
        const float m = wave_max(fabsf(yv));
        if ((threadIdx.x & 63) == 0)
            hmax[threadIdx.x >> 6] = m;
        __syncthreads();
        const uint32_t w2 = (threadIdx.x >> 7) * 2;
        const float mh = fmaxf(hmax[w2], hmax[w2 + 1]);
        int ex = 0;
        if (mh > 0.f && mh <= 3.0e38f)
            frexpf(mh, &ex);
        const float sc = mh > 0.f ? ldexpf(1.0f, ex - 14) : 1.0f;
        if ((threadIdx.x & 127) == 0)
            a.y_bscale[(size_t)t * (a.dim >> 7) + (ch >> 7)] = sc;
        _Float16 hh, ll;
        split_f16(yv * (1.0f / sc), hh, ll);
        const size_t o = blocked_index(t, ch, a.dim);
        reinterpret_cast<_Float16 *>(a.y_hi)[o] = hh;
        reinterpret_cast<_Float16 *>(a.y_lo)[o] = ll;
    } else {
        a.y[(size_t)t * a.dim + ch] = yv;
    }
    if (t + 1 == a.T) {
        a.state_next[ch * 2] = s1;
        a.state_next[ch * 2 + 1] = bx;
    }
}

// ------------------------------------------------------------------ attention

// Per token: q heads and k heads RMS-normed over head_dim and NEOX-rotated at
// position start + t (table row), q written back, K and V rounded to binary16 and
// stored in the cache (lfm.rs:360-393).  One wave per head.
// Wave w takes q heads w + 4i (heads <= 32) and kv heads w + 4j (kv <= 8).  Every
// value it needs (all split-K slices of its q, k and v heads, the norm weights and
// the position's rotation) is loaded before the first is used: a per-head loop of
// load, reduce and store waited for each head in turn (the stores may alias the
// next head's loads).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_rope_kv_prefill(const RopeKvArgs a)
{
    const uint32_t t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (t >= a.T)
        return;
    const uint32_t dim = a.heads * 64, hdkv = a.kv * 64, W = dim + 2 * hdkv, pos = a.start + t;
    const size_t rowo = (size_t)t * W;
    float *row = a.qkv + rowo;
    const float *cs = a.rope + (size_t)pos * 64;
    const uint32_t p = lane & 31;
    const float c = cs[2 * p], s = cs[2 * p + 1], qw = a.q_norm[lane], kw = a.k_norm[lane];
    size_t off[12];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        off[i] = min(wave + 4 * i, a.heads - 1) * 64 + lane;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t kh = min(wave + 4 * j, a.kv - 1);
        off[8 + j] = dim + kh * 64 + lane;
        off[10 + j] = dim + hdkv + kh * 64 + lane;
    }
    float v[12];
    slice_sums<12, 4>(a.src + rowo, (size_t)a.T * W, a.ksplit, off, v);
    auto norm_rope = [&](float x, float w) {
        const float ss = wave_sum(x * x);
        const float inv = 1.0f / sqrtf(ss / 64.0f + a.eps);
        x *= inv * w;
        const float2v xh = wave_halves(x);
        const float other = lane < 32 ? xh[1] : xh[0];
        return lane < 32 ? x * c - other * s : other * s + x * c;
    };
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t h = wave + 4 * i;
        if (h < a.heads) // uniform
            row[h * 64 + lane] = norm_rope(v[i], qw);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t kh = wave + 4 * j;
        if (kh < a.kv) { // uniform
            const float r = norm_rope(v[8 + j], kw);
            const size_t o = ((size_t)kh * a.ctx + pos) * 64 + lane;
            a.kcache[o] = __builtin_bit_cast(uint16_t, (_Float16)r);
            a.vcache[o] = __builtin_bit_cast(uint16_t, (_Float16)v[10 + j]);
        }
    }
}

// Causal attention (lfm.rs:395-437) on the matrix cores.  A workgroup takes 32
// queries of one kv head; wave w is q head kh*G + w.  Keys stream in blocks of
// 32 through double-buffered LDS (K rows, V transposed), shared by the G heads.
// Per block a wave computes S^T = K Q^T (keys x queries) with
// v_mfma_f32_32x32x16_f16 on q split into binary16 hi + lo (K is binary16 in the
// cache), so each lane holds one query's 16 scores: the online softmax (running
// max m, sum l, fp32) needs only in-lane work and one swap across lane halves.
// The lane's probabilities, split hi + lo, feed O^T += V^T P^T on the same
// 32x32x16 MFMA: for keys 16 G .. 16 G + 15, lane slot j of both operands is key
// 16 G + 8 (j / 4) + 4 (lane / 32) + j % 4, i.e. the lane's score items 8 G .. 8 G
// + 7 and two 4-key pieces of each V^T row (the 32x32x8 form, which takes as long
// per instruction, would need twice the instructions).  Only blocks that reach past
// the tile's first query position are masked; the rescale of O is skipped when no
// lane's running maximum changed (a factor of exactly 1).  out = O / l.
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef float floatx16a __attribute__((ext_vector_type(16)));
#define FA_Q 32    // queries per workgroup
#define FA_K 32    // keys per block
#define FA_KROW 72 // halves per K row in LDS (64 + 8)
#define FA_VROW 36 // halves per transposed-V row in LDS (32 + 4)
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_attn_prefill(const AttnPrefillArgs a)
{
    const uint32_t ntile = (a.T + FA_Q - 1) / FA_Q;
    const uint32_t kh = blockIdx.y, G = a.heads / a.kv, dim = a.heads * 64, hdkv = a.kv * 64,
                   stride = dim + 2 * hdkv;
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lq = lane & 31,
                   lh = lane >> 5;
    __shared__ __attribute__((aligned(16))) _Float16 Ks[2][FA_K * FA_KROW];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[2][64 * FA_VROW];
    const bool active = wave < G;
    const uint32_t h = kh * G + (active ? wave : 0);
    // q fragments (B operand, 16 keys-dims steps): lane holds query lq, dims ks*16 + 8*lh + i.
    // Scores are kept in log2 units (q scaled by scale * log2 e), so the softmax
    // exponentials are single v_exp_f32 (2^x): 2^(s2 - m2) = e^(s - m).
    const float qscale = a.scale * 1.4426950408889634f;
    // The longest (latest) query tiles are dispatched first.  Paired: workgroup b
    // runs tile ntile - 1 - b and then tile b (every workgroup near ntile + 1 key
    // blocks, so the causal triangle does not leave the long tiles sharing their
    // SIMDs with short ones); the middle tile of an odd count runs once.
    for (uint32_t pass = 0; pass < (a.paired ? 2u : 1u); ++pass) {
        const uint32_t tile = pass ? blockIdx.x : a.paired ? ntile - 1 - blockIdx.x : gridDim.x - 1 - blockIdx.x;
        if (tile >= ntile || (pass && tile >= ntile - 1 - blockIdx.x)) // uniform
            break;
        const uint32_t t0 = tile * FA_Q;
        const uint32_t tq = t0 + lq;
        half8 qh[4], ql[4];
        {
            const float *qrow = a.qkv + (size_t)(tq < a.T ? tq : a.T - 1) * stride + h * 64;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const float4 v0 = *reinterpret_cast<const float4 *>(qrow + ks * 16 + 8 * lh);
                const float4 v1 = *reinterpret_cast<const float4 *>(qrow + ks * 16 + 8 * lh + 4);
                const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float x = v[i] * qscale;
                    qh[ks][i] = (_Float16)x;
                    ql[ks][i] = (_Float16)(x - (float)qh[ks][i]);
                }
            }
        }
        const uint32_t qpos = a.start + tq; // causal limit of this lane's query
        const uint32_t tmax = min(t0 + FA_Q, a.T) - 1;
        // key blocks [kb_lo, kb_hi) of this workgroup: all the causal ones, or one range
        const uint32_t nblk_all = (a.start + tmax) / FA_K + 1;
        const uint32_t kb_lo = a.kb_per ? blockIdx.z * a.kb_per : 0;
        const uint32_t kb_hi = a.kb_per ? min(nblk_all, kb_lo + a.kb_per) : nblk_all;
        const uint32_t nblk = kb_hi > kb_lo ? kb_hi - kb_lo : 0;
        // staging: thread -> key row tid / 8, dims (tid % 8) * 8 .. +7
        const uint32_t sr = tid >> 3, sp = (tid & 7) * 8;
        const uint16_t *kg = a.kcache + (size_t)kh * a.ctx * 64;
        const uint16_t *vg = a.vcache + (size_t)kh * a.ctx * 64;
        auto load_kv = [&](uint32_t blk, uint4 &kr, uint4 &vr) { // blk counts from kb_lo
            const uint32_t pos = min((kb_lo + blk) * FA_K + sr, a.ctx - 1);
            kr = *reinterpret_cast<const uint4 *>(kg + (size_t)pos * 64 + sp);
            vr = *reinterpret_cast<const uint4 *>(vg + (size_t)pos * 64 + sp);
        };
        auto store_kv = [&](uint32_t buf, uint4 kr, uint4 vr) {
            *reinterpret_cast<uint4 *>(&Ks[buf][sr * FA_KROW + sp]) = kr;
            const uint16_t *v16 = reinterpret_cast<const uint16_t *>(&vr);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                reinterpret_cast<uint16_t *>(Vt[buf])[(sp + i) * FA_VROW + sr] = v16[i];
        };
        floatx16a o0, o1;
#pragma unroll
        for (int e = 0; e < 16; ++e)
            o0[e] = 0.f, o1[e] = 0.f;
        float m = -INFINITY, l = 0.f;
        uint4 kr, vr;
        if (nblk > 0) {
            load_kv(0, kr, vr);
            store_kv(0, kr, vr);
        }
        if (nblk > 1)
            load_kv(1, kr, vr);
        __syncthreads();
        for (uint32_t blk = 0; blk < nblk; ++blk) {
            const uint32_t buf = blk & 1;
            if (active) {
                // S^T[key][query] for the block's 32 keys
                floatx16a sacc;
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    sacc[e] = 0.f;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const half8 kf = *reinterpret_cast<const half8 *>(&Ks[buf][lq * FA_KROW + ks * 16 + 8 * lh]);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qh[ks], sacc, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, ql[ks], sacc, 0, 0, 0);
                }
                // lane's items: keys 8*(e/4) + 4*lh + e%4 of the block, query lq.  A block
                // that ends before the tile's first query position needs no mask; its
                // scores are finite, and so is the new maximum.
                const bool diag = (kb_lo + blk + 1) * FA_K > a.start + t0;
                float bm = -INFINITY;
                if (diag) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const uint32_t kpos = (kb_lo + blk) * FA_K + 8 * (e / 4) + 4 * lh + (e % 4);
                        if (kpos > qpos)
                            sacc[e] = -INFINITY;
                    }
                }
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    bm = fmaxf(bm, sacc[e]);
                const float2v bh = wave_halves(bm);
                bm = fmaxf(bh[0], bh[1]);
                const float mn = fmaxf(m, bm);
                const float r = m > -INFINITY ? __builtin_amdgcn_exp2f(m - mn) : 0.f;
                // masked scores are -inf and 2^-inf = 0; a query with no unmasked key
                // yet (a key range wholly past it) has mn = -inf and subtracts 0
                const float mz = mn > -INFINITY ? mn : 0.f;
                float ps = 0.f;
                half8 phi[2], plo[2];
#pragma unroll
                for (int e = 0; e < 16; e += 2) {
                    const float p0 = __builtin_amdgcn_exp2f(sacc[e] - mz), p1 = __builtin_amdgcn_exp2f(sacc[e + 1] - mz);
                    ps += p0;
                    ps += p1;
                    const half2v hp = __builtin_convertvector((float2v){p0, p1}, half2v);
                    const float2v hb = __builtin_convertvector(hp, float2v);
                    const half2v lp = __builtin_convertvector((float2v){p0 - hb[0], p1 - hb[1]}, half2v);
                    phi[e / 8][e % 8] = hp[0];
                    phi[e / 8][e % 8 + 1] = hp[1];
                    plo[e / 8][e % 8] = lp[0];
                    plo[e / 8][e % 8 + 1] = lp[1];
                }
                const float2v sh = wave_halves(ps);
                ps = sh[0] + sh[1];
                l = l * r + ps;
                m = mn;
                if (__ballot(r != 1.0f) != 0) {
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        o0[e] *= r, o1[e] *= r;
                }
                // O^T[dim][query] += V^T[dim][key] P^T[key][query], keys in groups of 16
#pragma unroll
                for (int G = 0; G < 2; ++G) {
                    const half4v a0 = *reinterpret_cast<const half4v *>(&Vt[buf][lq * FA_VROW + 16 * G + 4 * lh]);
                    const half4v b0 = *reinterpret_cast<const half4v *>(&Vt[buf][lq * FA_VROW + 16 * G + 8 + 4 * lh]);
                    const half4v a1 = *reinterpret_cast<const half4v *>(&Vt[buf][(32 + lq) * FA_VROW + 16 * G + 4 * lh]);
                    const half4v b1 =
                        *reinterpret_cast<const half4v *>(&Vt[buf][(32 + lq) * FA_VROW + 16 * G + 8 + 4 * lh]);
                    const half8 v0 = {a0[0], a0[1], a0[2], a0[3], b0[0], b0[1], b0[2], b0[3]};
                    const half8 v1 = {a1[0], a1[1], a1[2], a1[3], b1[0], b1[1], b1[2], b1[3]};
                    o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v0, phi[G], o0, 0, 0, 0);
                    o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v0, plo[G], o0, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v1, phi[G], o1, 0, 0, 0);
                    o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(v1, plo[G], o1, 0, 0, 0);
                }
            }
            if (blk + 1 < nblk)
                store_kv(buf ^ 1, kr, vr);
            if (blk + 2 < nblk)
                load_kv(blk + 2, kr, vr);
            __syncthreads();
        }
        if (active && tq < a.T) {
            if (a.kb_per) { // this key range's softmax state, merged by k_attn_merge_split
                float *pp = a.part + (((size_t)blockIdx.z * a.T + tq) * a.heads + h) * 66;
                if (lh == 0) {
                    pp[0] = m;
                    pp[1] = l;
                }
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t d = 8 * (e / 4) + 4 * lh + (e % 4);
                    pp[2 + d] = o0[e];
                    pp[2 + 32 + d] = o1[e];
                }
            } else {
                const float rl = 1.0f / l;
                float *orow = a.out + (size_t)tq * dim + h * 64;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const uint32_t d = 8 * (e / 4) + 4 * lh + (e % 4);
                    orow[d] = o0[e] * rl;
                    orow[32 + d] = o1[e] * rl;
                }
            }
        }
    } // pass
}

// Combines the key ranges of a split prefill attention: for (query t, head h),
// out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s (scores in log2 units).
// Workgroup: one query, four heads (thread: head tid / 64, dim tid % 64).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_attn_merge_split(const AttnMergeSplitArgs a)
{
    const uint32_t t = blockIdx.x, h = blockIdx.y * 4 + (threadIdx.x >> 6), d = threadIdx.x & 63;
    if (t >= a.T || h >= a.heads)
        return;
    const size_t stride = (size_t)a.T * a.heads * 66;
    const float *pb = a.part + ((size_t)t * a.heads + h) * 66;
    const uint32_t n = a.nsplit;
    // the ranges in batches of 8, a batch's loads issued before its first use
    // (indexes clamped, the extra values unused): a load-use loop waited for each
    // range in turn
    float M = -INFINITY;
    for (uint32_t s0 = 0; s0 < n; s0 += 8) {
        float m[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            m[j] = pb[(size_t)min(s0 + j, n - 1) * stride];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < n)
                M = fmaxf(M, m[j]);
    }
    float num = 0.f, den = 0.f;
    for (uint32_t s0 = 0; s0 < n; s0 += 8) {
        float m[8], l[8], o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float *q = pb + (size_t)min(s0 + j, n - 1) * stride;
            m[j] = q[0];
            l[j] = q[1];
            o[j] = q[2 + d];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (s0 + j < n) {
                const float f = m[j] > -INFINITY ? __builtin_amdgcn_exp2f(m[j] - M) : 0.f;
                den += f * l[j];
                num += f * o[j];
            }
    }
    const float yv = num / den;
    if (a.y_hi) { // uniform (heads a multiple of 4): waves 2i, 2i + 1 hold half-block i
        __shared__ float hmax[4];
        const float m = wave_max(fabsf(yv));
        if (d == 0)
            hmax[threadIdx.x >> 6] = m;
        __syncthreads();
        const uint32_t w2 = (threadIdx.x >> 7) * 2, K = a.heads * 64, k = h * 64 + d;
        const float mh = fmaxf(hmax[w2], hmax[w2 + 1]);
        int ex = 0;
        if (mh > 0.f && mh <= 3.0e38f)
            frexpf(mh, &ex);
        const float sc = mh > 0.f ? ldexpf(1.0f, ex - 14) : 1.0f;
        if ((threadIdx.x & 127) == 0)
            a.y_bscale[(size_t)t * (K >> 7) + (k >> 7)] = sc;
        _Float16 hh, ll;
        split_f16(yv * (1.0f / sc), hh, ll);
        const size_t o = blocked_index(t, k, K);
        reinterpret_cast<_Float16 *>(a.y_hi)[o] = hh;
        reinterpret_cast<_Float16 *>(a.y_lo)[o] = ll;
        return;
    }
    a.out[(size_t)t * a.heads * 64 + h * 64 + d] = yv;
}

// ------------------------------------------------------------------ FFN pieces
// Router logits of a large call on the matrix cores (lfm.rs:599-607): logits[t][e] =
// sum_k W[e][k] xn[t][k], xn = RMSNorm(x_t) * ffn_norm, from the FFN input's split
// (binary16 hi + lo of xn / xscale[t], row-major, written before this kernel) and the
// router rows split once into hi + lo of W * 2^s (k_router_split; s puts max |W| in
// [2^13, 2^14), so the lo halves stay normal).  A workgroup takes 32 tokens; wave w
// sums the k-steps [w nks / 4, (w + 1) nks / 4) of 16 with three products per step
// (Wh Xh, Wh Xl, Wl Xh on v_mfma_f32_32x32x16_f16; Wl Xl is below 2^-22 of a term),
// the next step's fragments loaded during the current one's products, and wave 0
// adds the four partial tiles in order.  32 experts per pass (two passes for up to
// 64).  Lane l holds expert rows 8 (j / 4) + 4 (l / 32) + j % 4 of token l % 32.
extern "C" __global__ __launch_bounds__(64) void k_router_split(const RouterSplitArgs a)
{
    const uint32_t i = blockIdx.x * 64 + threadIdx.x;
    if (i >= a.n)
        return;
    _Float16 h, l;
    split_f16(a.w[i] * a.scale, h, l);
    a.hi[i] = __builtin_bit_cast(uint16_t, h);
    a.lo[i] = __builtin_bit_cast(uint16_t, l);
}

extern "C" __global__ __launch_bounds__(WG_THREADS) void k_router_mfma(const RouterMfmaArgs a)
{
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const uint32_t p = lane >> 5, lr = lane & 31, t0 = blockIdx.x * 32;
    if (t0 >= a.T)
        return;
    const uint32_t t = min(t0 + lr, a.T - 1), nks = a.K / 16;
    const uint32_t ks0 = wave * nks / 4, ks1 = (wave + 1) * nks / 4;
    __shared__ floatx16 part[4][64];
    const half8 *xh = reinterpret_cast<const half8 *>(a.x_hi) + ((size_t)t * a.K + 8 * p) / 8;
    const half8 *xl = reinterpret_cast<const half8 *>(a.x_lo) + ((size_t)t * a.K + 8 * p) / 8;
    for (uint32_t et = 0; et < a.E; et += 32) {
        const uint32_t e = min(et + lr, a.E - 1);
        const half8 *wh = reinterpret_cast<const half8 *>(a.w_hi) + ((size_t)e * a.K + 8 * p) / 8;
        const half8 *wl = reinterpret_cast<const half8 *>(a.w_lo) + ((size_t)e * a.K + 8 * p) / 8;
        floatx16 acc;
#pragma unroll
        for (int j = 0; j < 16; ++j)
            acc[j] = 0.f;
        half8 bh = xh[2 * ks0], bl = xl[2 * ks0], ah = wh[2 * ks0], al = wl[2 * ks0];
        for (uint32_t ks = ks0; ks < ks1; ++ks) {
            const uint32_t kn = min(ks + 1, ks1 - 1); // the next step's fragments (the last re-reads its own)
            const half8 nbh = xh[2 * kn], nbl = xl[2 * kn], nah = wh[2 * kn], nal = wl[2 * kn];
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, acc, 0, 0, 0);
            bh = nbh, bl = nbl, ah = nah, al = nal;
        }
        part[wave][lane] = acc;
        __syncthreads();
        if (wave == 0 && t0 + lr < a.T) {
            floatx16 s = part[0][lane];
            s += part[1][lane];
            s += part[2][lane];
            s += part[3][lane];
            const float f = a.xscale[t0 + lr] * a.unscale;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t ee = et + 8 * (j / 4) + 4 * p + (j % 4);
                if (ee < a.E)
                    a.logits[(size_t)(t0 + lr) * a.E + ee] = s[j] * f;
            }
        }
        __syncthreads();
    }
}

// Router logits for calls of up to 128 tokens: one workgroup per (expert, token)
// (grid n_expert x T), thread tid covering inputs 8 tid .. 8 tid + 7 of the
// token's x . w (dim <= 2048), so the workgroup also sums x^2 for the RMSNorm
// scale; logits = inv * dot.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_router_prefill_small(const RouterPrefillArgs a)
{
    __shared__ float red[2][4];
    const uint32_t e = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    if (e >= a.n_expert || t >= a.T)
        return;
    const float *x = a.x + (size_t)t * a.dim, *w = a.w + (size_t)e * a.dim;
    float ss = 0.f, dot = 0.f;
    for (uint32_t k = tid * 8; k < a.dim; k += WG_THREADS * 8) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 x4 = *reinterpret_cast<const float4 *>(x + k + 4 * h);
            const float4 n4 = *reinterpret_cast<const float4 *>(a.norm_w + k + 4 * h);
            const float4 w4 = *reinterpret_cast<const float4 *>(w + k + 4 * h);
            ss += x4.x * x4.x + x4.y * x4.y + x4.z * x4.z + x4.w * x4.w;
            dot = fmaf(x4.x * n4.x, w4.x, dot);
            dot = fmaf(x4.y * n4.y, w4.y, dot);
            dot = fmaf(x4.z * n4.z, w4.z, dot);
            dot = fmaf(x4.w * n4.w, w4.w, dot);
        }
    }
    ss = wave_sum(ss);
    dot = wave_sum(dot);
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = ss;
        red[1][tid >> 6] = dot;
    }
    __syncthreads();
    if (tid == 0) {
        const float tss = ((red[0][0] + red[0][1]) + red[0][2]) + red[0][3];
        const float td = ((red[1][0] + red[1][1]) + red[1][2]) + red[1][3];
        a.logits[(size_t)t * a.n_expert + e] = td / sqrtf(tss / (float)a.dim + a.eps);
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
// 1024 threads, so that a 3840-token call takes four passes of ballots and
// barriers instead of fifteen.
#define RG_THREADS 1024
extern "C" __global__ __launch_bounds__(RG_THREADS) void k_route_group(const RouteGroupArgs a)
{
    constexpr uint32_t NWV = RG_THREADS / 64;
    const uint32_t e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ uint32_t wave_cnt[NWV];
    __shared__ uint32_t base;
    if (tid == 0)
        base = 0;
    __syncthreads();
    for (uint32_t t0 = 0; t0 < a.T; t0 += RG_THREADS) {
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
            if (a.pos)
                a.pos[t * 4 + rank_of_e] = off + before;
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t sum = base;
            for (uint32_t w = 0; w < NWV; ++w)
                sum += wave_cnt[w];
            base = sum;
        }
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
    // thread: 4 consecutive k of token t; every rank's loads issued together
    const uint32_t k = (blockIdx.x * WG_THREADS + threadIdx.x) * 4, t = blockIdx.y;
    if (k >= a.dim || t >= a.T)
        return;
    float4 dv[4];
    float wv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const bool on = r < (int)a.n_used;
        dv[r] = on ? *reinterpret_cast<const float4 *>(a.d + ((size_t)t * 4 + r) * a.dim + k)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[r] = on ? a.wsel[(size_t)t * 4 + r] : 0.f;
    }
    float4 *xp = reinterpret_cast<float4 *>(a.x + (size_t)t * a.dim + k);
    const float4 x0 = *xp;
    float4 sm = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (r < (int)a.n_used) {
            sm.x = sm.x + dv[r].x * wv[r];
            sm.y = sm.y + dv[r].y * wv[r];
            sm.z = sm.z + dv[r].z * wv[r];
            sm.w = sm.w + dv[r].w * wv[r];
        }
    *xp = make_float4(x0.x + sm.x, x0.y + sm.y, x0.z + sm.z, x0.w + sm.w);
}

// The expert down projection's K slices and the combine in one pass (split-K
// calls): d = sum_s part[s] in slice order, then k_combine_prefill's
// x += ((0 + d_0 w_0) + d_1 w_1) + ... in rank order, no contraction.
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_reduce_combine(const ReduceCombineArgs a)
{
#pragma clang fp contract(off)
    const uint32_t k = blockIdx.x * WG_THREADS + threadIdx.x, t = blockIdx.y;
    if (k >= a.dim || t >= a.T)
        return;
    const size_t slice = (size_t)a.T * 4 * a.dim;
    float *x = a.x + (size_t)t * a.dim + k;
    const float x0 = *x;
    float w[4], d[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r)
        w[r] = a.wsel[(size_t)t * 4 + r];
    // the four ranks' slices together (ranks >= n_used are read and not used)
    const size_t D = a.dim;
    slice_sums<4>(a.part + (size_t)t * 4 * a.dim + k, slice, a.ksplit, {0, D, 2 * D, 3 * D}, d);
    float sm = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (r < (int)a.n_used)
            sm = sm + d[r] * w[r];
    *x = x0 + sm;
}

// Token embeddings of T ids (lfm.rs:310-320): row ids[t] of the Q6_K table,
// dequantized exactly; one wave per row (8 lanes per 256-wide block).
extern "C" __global__ __launch_bounds__(WG_THREADS) void k_embed_rows(const EmbedRowsArgs a)
{
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (a.st && blockIdx.x == 0 && threadIdx.x == 0) { // uniform per workgroup
        DevState *st = a.st;
        st->tok = a.ids ? a.ids[0] : a.ids_inline[0];
        st->pos = a.start;
        st->halt = 0;
        st->step = 0;
        st->eos = ~0u;
        st->cursor = 0;
        st->n_ids = a.T;
        st->last_token = 0;
        st->last_value = 0.f;
        st->fault = 0;
#pragma unroll
        for (int i = 0; i < 5; ++i)
            st->pad[i] = 0;
    }
    if (t >= a.T)
        return;
    const uint32_t tok = a.ids ? a.ids[t] : a.ids_inline[t];
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
