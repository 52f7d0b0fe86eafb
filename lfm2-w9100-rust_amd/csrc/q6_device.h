// q6_device.h -- device-side access to the Q6_K plane layout (kargs.h), shared by
// the decode (lfm_kernels.hip) and prefill (lfm_prefill.hip) code objects.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kargs.h"

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

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
// The ql / qh planes (92 % of the bytes) are streamed: a decode step reads each
// weight byte once, and a step's 1.3 GB do not fit the Infinity Cache, so their
// loads are non-temporal (a plain read of 110 MiB measures 5.6 TB/s with cached
// loads, 6.0 TB/s non-temporal; 512 MiB: 6.3 and 7.0 TB/s).  The scale and d
// planes stay cached by default: neighbouring rows share their cache lines (16 B
// of d per row), which measured faster for the decode step as a whole; the tied
// head, which streams 110 MB in one launch, is faster with every plane streamed
// (StreamAll).
template <bool StreamAll = false>
__device__ __forceinline__ Lane load_lane(const Q6T &t, uint32_t row, uint32_t b, uint32_t c)
{
    const size_t nblk = (size_t)t.rows * t.nb;
    const size_t blk = (size_t)row * t.nb + b;
    const u32x4_t q = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(t.base + blk * 128 + c * 16));
    const u32x2_t h = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(t.base + nblk * 128 + blk * 64 + c * 8));
    const uint32_t *scp = reinterpret_cast<const uint32_t *>(t.base + nblk * 192 + blk * 16 + (c >> 1) * 4);
    const uint16_t *dp = reinterpret_cast<const uint16_t *>(t.base + nblk * 208) + blk;
    Lane w;
    w.ql = make_uint4(q.x, q.y, q.z, q.w);
    w.qh = make_uint2(h.x, h.y);
    if constexpr (StreamAll) {
        w.sc = __builtin_nontemporal_load(scp);
        w.d = __builtin_nontemporal_load(dp);
    } else {
        w.sc = *scp;
        w.d = *dp;
    }
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

