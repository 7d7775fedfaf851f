// rows.h — vectorised per-row int8 quantization (internal header).
//
// The per-token quantizers (quant.hip) and the producer-fused ones
// (producer.hip) all reduce one row to its absmax and then quantize it.  Rows
// are short (a head of 64 or 128 elements, a model row of 1–8K), so one lane
// per element leaves most of a wave's load slots empty.  Here each lane owns
// 16-byte chunks of a row instead: a row of C chunks is spread over
// L = min(C, 64) lanes (L a power of two) with C / L chunks per lane, so a
// wave holds 64 / L rows, loads are 16 bytes per lane and the row reductions
// are shuffles inside an aligned lane group.  Shapes that do not split this
// way keep the one-element-per-lane kernels.
#pragma once

#include <type_traits>

#include "int8k_common.h"

namespace int8k {

// Elements of a dtype per 16-byte chunk.
template <int DT>
struct Vec {
    static constexpr int W = DT == INT8K_DTYPE_F32 ? 4 : 8;
};

// At most this many chunks per lane (a row of 64 * 16 chunks = 16 KiB).
constexpr int kMaxChunksPerLane = 16;

// How a row of `cols` elements maps onto lanes: 1 << lg lanes, nc chunks each.
struct RowShape {
    int lg = 0, nc = 0;
    bool ok = false;
};

inline RowShape row_shape(int cols, int dtype) {
    RowShape r;
    const int w = dtype == INT8K_DTYPE_F32 ? 4 : 8;
    if (cols <= 0 || cols % w) return r;
    const int c = cols / w;
    if (c <= 64) {
        if (c & (c - 1)) return r;
        while ((1 << r.lg) < c) ++r.lg;
        r.nc = 1;
    } else {
        if (c % 64 || c / 64 > kMaxChunksPerLane) return r;
        r.lg = 6;
        r.nc = c / 64;
    }
    r.ok = true;
    return r;
}

// Chunks per lane of a kernel instance: NC > 0 is a compile-time count (no
// guards around the loads); NC = 0 means a runtime nc <= kMaxChunksPerLane.
template <int NC>
constexpr int chunk_slots() {
    return NC > 0 ? NC : kMaxChunksPerLane;
}

// Calls f(std::integral_constant<int, NC>) with NC = nc for the common counts
// 1, 2, 4, 8, 16, and NC = 0 (runtime count) otherwise.
template <typename F>
inline void with_chunks(int nc, F&& f) {
    switch (nc) {
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        case 4: f(std::integral_constant<int, 4>{}); break;
        case 8: f(std::integral_constant<int, 8>{}); break;
        case 16: f(std::integral_constant<int, 16>{}); break;
        default: f(std::integral_constant<int, 0>{});
    }
}

// Calls f(std::integral_constant<int, DT>) for a dtype code.
template <typename F>
inline void with_dtype(int dtype, F&& f) {
    switch (dtype) {
        case INT8K_DTYPE_F16: f(std::integral_constant<int, INT8K_DTYPE_F16>{}); break;
        case INT8K_DTYPE_BF16: f(std::integral_constant<int, INT8K_DTYPE_BF16>{}); break;
        default: f(std::integral_constant<int, INT8K_DTYPE_F32>{});
    }
}

// Makes the compiler treat a chunk as rewritten, so values unpacked from it
// before this point are not kept live across it (they are cheaper to unpack
// again than to hold in 2 W registers per chunk).
__device__ __forceinline__ void reload_barrier(uint4& w) {
    asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));
}

template <int DT>
__device__ __forceinline__ void unpack_chunk(const uint4& w, float (&v)[Vec<DT>::W]) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (DT == INT8K_DTYPE_F32) {
            v[i] = __uint_as_float(d[i]);
        } else if constexpr (DT == INT8K_DTYPE_F16) {
            v[2 * i] = __half2float(__ushort_as_half((unsigned short)(d[i] & 0xffffu)));
            v[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(d[i] >> 16)));
        } else {
            v[2 * i] = __uint_as_float(d[i] << 16);
            v[2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
        }
    }
}

// Reduction over the aligned group of 1 << lg lanes that holds one row; every
// lane of the group gets the result.
template <typename Op>
__device__ __forceinline__ float row_reduce(float v, int lg, Op op) {
#pragma unroll
    for (int k = 0; k < 6; ++k)
        if (k < lg) v = op(v, __shfl_xor(v, 1 << k));
    return v;
}

// The per-token quantizer's code: rn(clamp(y / s, -128, 127)) with a true division.
__device__ __forceinline__ int quant_code(float y, float s) {
    return (int)__builtin_rintf(fminf(fmaxf(y / s, -128.f), 127.f));
}

// W codes of one chunk, stored as W consecutive bytes (W = 4 or 8): the same
// codes as quant_code(v, s) for every input, without a division.  With
// inv = 1/s correctly rounded, t = v * inv, r = v - t s (exact, one FMA) and
// q = t + r inv is the correctly rounded quotient v / s (Markstein's
// correction step; checked against true division on 1.2e10 random quantizer
// inputs, s = max(amax, 1e-8)/127 and |v| <= amax), so rint(clamp(q)) is the
// code.  A NaN element gives NaN on both paths.  An infinite element makes s
// infinite and inv zero: the step then uses 0 for s, so q = t = v * 0, which is
// v / s for finite v and NaN for infinite v, as the division gives.  No
// branch: a branch here, even one never taken, split the quantizers' load and
// store scheduling and cost them about 30%.
template <int W>
__device__ __forceinline__ void store_codes(const float (&v)[W], float s, float inv, int8_t* dst) {
#pragma clang fp contract(off)
    const float s_step = inv != 0.f ? s : 0.f;
    float q[W];
#pragma unroll
    for (int i = 0; i < W; ++i) {
        const float t = v[i] * inv;
        q[i] = __builtin_fmaf(__builtin_fmaf(-t, s_step, v[i]), inv, t);
    }
    uint32_t b[W / 4];
#pragma unroll
    for (int j = 0; j < W / 4; ++j) {
        b[j] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = (int)__builtin_rintf(fminf(fmaxf(q[4 * j + i], -128.f), 127.f));
            b[j] |= ((uint32_t)c & 0xffu) << (8 * i);
        }
    }
    if constexpr (W == 8)
        *reinterpret_cast<uint2*>(dst) = make_uint2(b[0], b[1]);
    else
        *reinterpret_cast<uint32_t*>(dst) = b[0];
}

}  // namespace int8k
