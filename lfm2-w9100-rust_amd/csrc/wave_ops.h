// wave_ops.h -- wave64 reductions and the MoE routing rule, shared by the
// decode (lfm_kernels.hip) and prefill (lfm_prefill.hip) code objects.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kargs.h"

// Wave-wide reductions with DPP lane moves (quad permutes, row shifts, row
// broadcasts: all VALU, no LDS round trips); the total lands in lane 63 and
// is broadcast with readlane.  Every lane of the wave must be active.
template <int CTRL> __device__ __forceinline__ float dpp_mov(float v, float old)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, v), CTRL,
                                                                 0xf, 0xf, false));
}

__device__ __forceinline__ float lane63(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp_mov<0xb1>(v, 0.f);  // quad_perm [1,0,3,2]
    v += dpp_mov<0x4e>(v, 0.f);  // quad_perm [2,3,0,1]
    v += dpp_mov<0x114>(v, 0.f); // row_shr:4
    v += dpp_mov<0x118>(v, 0.f); // row_shr:8
    v += dpp_mov<0x142>(v, 0.f); // row_bcast:15
    v += dpp_mov<0x143>(v, 0.f); // row_bcast:31
    return lane63(v);
}

// Sum over each group of four lanes, in all four lanes.
__device__ __forceinline__ float quad_sum(float v)
{
    v += dpp_mov<0xb1>(v, 0.f); // quad_perm [1,0,3,2]
    v += dpp_mov<0x4e>(v, 0.f); // quad_perm [2,3,0,1]
    return v;
}

// Sums over each half of the wave: lanes 0..31 in lane 31, lanes 32..63 in
// lane 63 (the first five steps of wave_sum).
__device__ __forceinline__ float half_wave_sum(float v)
{
    v += dpp_mov<0xb1>(v, 0.f);
    v += dpp_mov<0x4e>(v, 0.f);
    v += dpp_mov<0x114>(v, 0.f);
    v += dpp_mov<0x118>(v, 0.f);
    v += dpp_mov<0x142>(v, 0.f);
    return v;
}

// N independent wave sums, their DPP steps interleaved so that each step's
// wait states are filled by the other sums (results in every lane).
template <int N> __device__ __forceinline__ void wave_sums(float *v)
{
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0xb1>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x4e>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x114>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x118>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x142>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x143>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] = lane63(v[i]);
}

// Half-wave form of wave_sums: lanes 0..31 summed in lane 31, 32..63 in 63.
template <int N> __device__ __forceinline__ void half_wave_sums(float *v)
{
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0xb1>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x4e>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x114>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x118>(v[i], 0.f);
#pragma unroll
    for (int i = 0; i < N; ++i)
        v[i] += dpp_mov<0x142>(v[i], 0.f);
}

typedef float float2v __attribute__((ext_vector_type(2)));
// v of lanes 0..31 and of lanes 32..63, each in both wave halves (lane l sees its
// own value and lane l ^ 32's): one v_permlane32_swap, a VALU lane move (a
// ds_bpermute shuffle goes through the LDS).  The results are copied out of the
// returned pair before the bit casts: __builtin_bit_cast of an element of it
// read element 0 for both.
__device__ __forceinline__ float2v wave_halves(float v)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t lo = r[0], hi = r[1];
    return {__builtin_bit_cast(float, lo), __builtin_bit_cast(float, hi)};
}

__device__ __forceinline__ float wave_max(float v)
{
    v = fmaxf(v, dpp_mov<0xb1>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x4e>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x114>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x118>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x142>(v, -INFINITY));
    v = fmaxf(v, dpp_mov<0x143>(v, -INFINITY));
    return lane63(v);
}

// MoE routing of one token (lfm.rs:613-637, resident.rs:58-99), computed by
// every wave from the router logits: p = sigmoid(logit), score = p + bias.
// Round k takes the largest remaining score, the lowest expert id among equal
// scores (the order of a stable descending sort); the n_used picks are
// weighted p / max(sum in rank order, 2^-14).  NaN scores are never picked
// while a number remains; the ids are always valid experts.  Results are
// wave-uniform scalars (small arrays would be placed in memory).
struct Routed {
    uint32_t id0, id1, id2, id3;
    float w0, w1, w2, w3;
    __device__ __forceinline__ uint32_t id(uint32_t k) const
    {
        return k == 0 ? id0 : k == 1 ? id1 : k == 2 ? id2 : id3;
    }
    __device__ __forceinline__ float w(uint32_t k) const
    {
        return k == 0 ? w0 : k == 1 ? w1 : k == 2 ? w2 : w3;
    }
};

__device__ __forceinline__ float lane_f32(float v, uint32_t j)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)j));
}

// The lane's router logit and bias (lane < n_expert), loaded apart from the
// selection so that a kernel can issue them before its other loads.
struct RouteIn {
    float lg, bias;
};

__device__ __forceinline__ RouteIn route_load(const Route &r)
{
    const uint32_t lane = threadIdx.x & 63;
    RouteIn in = {0.f, 0.f};
    if (lane < r.n_expert) {
        in.lg = r.logits[lane];
        in.bias = r.bias[lane];
    }
    return in;
}

// Decode form: every lane loads (the index clamped to a valid expert; lanes
// past n_expert are masked by wave_route), with no branch around the loads.
// `alt` (>= 64 floats) stands in for absent logits / bias (dense layers).
__device__ __forceinline__ RouteIn route_load_all(const Route &r, const float *alt)
{
    const uint32_t j = min(threadIdx.x & 63, r.n_expert - 1);
    const float *lg = r.logits ? r.logits : alt;
    const float *bs = r.bias ? r.bias : alt;
    return RouteIn{lg[j], bs[j]};
}

// Order-preserving integer key of a float: for numbers, a < b exactly when
// key(a) < key(b) (+0 and -0 are made equal first).  Integer maxima need no
// NaN handling and fold into single DPP instructions.
__device__ __forceinline__ int float_key(float v)
{
    const int b = __float_as_int(v + 0.0f);
    return b ^ ((b >> 31) & 0x7FFFFFFF);
}

template <int CTRL> __device__ __forceinline__ int dpp_imax(int v)
{
    const int o = __builtin_amdgcn_update_dpp((int)0x80000000, v, CTRL, 0xf, 0xf, false);
    return max(v, o);
}

__device__ __forceinline__ int wave_max_i(int v)
{
    v = dpp_imax<0xb1>(v);
    v = dpp_imax<0x4e>(v);
    v = dpp_imax<0x114>(v);
    v = dpp_imax<0x118>(v);
    v = dpp_imax<0x142>(v);
    v = dpp_imax<0x143>(v);
    return __builtin_amdgcn_readlane(v, 63);
}

// The ids of the n_used picks and their probabilities (weights before the
// normalization of route_normalize).  Selection on integer keys of the
// scores: removed experts and lanes past n_expert take the lowest key, NaN
// scores the next (below every number), so numbers rank exactly as floats.
// sigmoid(logit) with the hardware exp2 / reciprocal (a few ulp).
__device__ __forceinline__ float route_prob(float lg)
{
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(lg * -1.44269504088896341f));
}

// The selection score p + bias (lfm.rs:613-622) that the picks are ranked by.
__device__ __forceinline__ float route_score(const RouteIn in)
{
    return route_prob(in.lg) + in.bias;
}

__device__ __forceinline__ Routed wave_route_ids(const Route &r, const RouteIn in)
{
    const uint32_t lane = threadIdx.x & 63;
    const bool valid = lane < r.n_expert;
    float prob = 0.f;
    int key = (int)0x80000000;
    if (valid) {
        prob = route_prob(in.lg);
        const float score = prob + in.bias;
        key = score == score ? float_key(score) : (int)0x80000001;
    }
    uint32_t id[4];
    float p[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        id[k] = 0;
        p[k] = 0.f;
        if ((uint32_t)k < r.n_used) {
            const int best = wave_max_i(key);
            const uint64_t m = __ballot(valid && key == best);
            const uint32_t e = m ? (uint32_t)__ffsll((long long)m) - 1u : 0u;
            id[k] = e;
            p[k] = lane_f32(prob, e);
            if (lane == e)
                key = (int)0x80000000;
        }
    }
    Routed o;
    o.id0 = id[0], o.id1 = id[1], o.id2 = id[2], o.id3 = id[3];
    o.w0 = p[0], o.w1 = p[1], o.w2 = p[2], o.w3 = p[3];
    return o;
}

// Weights p / max(sum of the picks' p in rank order, 2^-14).
__device__ __forceinline__ void route_normalize(Routed &o, uint32_t n_used)
{
    float wsum = 0.f;
    wsum = wsum + o.w0;
    if (n_used > 1)
        wsum = wsum + o.w1;
    if (n_used > 2)
        wsum = wsum + o.w2;
    if (n_used > 3)
        wsum = wsum + o.w3;
    if (wsum < 6.103515625e-5f)
        wsum = 6.103515625e-5f;
    o.w0 = o.w0 / wsum, o.w1 = o.w1 / wsum, o.w2 = o.w2 / wsum, o.w3 = o.w3 / wsum;
}

__device__ __forceinline__ Routed wave_route(const Route &r, const RouteIn in)
{
    Routed o = wave_route_ids(r, in);
    route_normalize(o, r.n_used);
    return o;
}

__device__ __forceinline__ Routed wave_route(const Route &r)
{
    return wave_route(r, route_load(r));
}
