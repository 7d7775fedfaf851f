// producer.hip — quantize-on-emit kernels for the ops that feed the INT8 attention and MLP.
//
// In the reference's transformer block every INT8 kernel input is produced by a
// separate eager quantization after the fp16 producer (bench/bench_block.py:59-63,
// 104-110, 119-121, 138-139): LayerNorm -> fp16 -> per-token quant for the MLP
// input, and QKV projection -> split heads -> .contiguous() -> per-token quant of
// Q, K and V.  These kernels do each of those chains in one pass:
//
//   layernorm_quant_kernel : y = LN(x) [fp32, biased variance, eps inside the
//       rsqrt, optional affine], rounded to the input dtype (what F.layer_norm
//       returns), then the per-token quantizer on that rounded y.  Optionally y
//       itself is written too.
//   quant_heads_kernel     : x [B, S, parts, H, Dh] (the QKV projection output
//       viewed by part and head) -> for each part, int8 [B, H, S, Dh] and fp32
//       scales [B, H, S]: per-token quantization over Dh, the layout the attention
//       kernels read.
//
// The quantizer is the one of quant.hip: s = max(amax, 1e-8) / 127,
// q = rn(clamp(y / s, -128, 127)) with a true division.
#include <algorithm>

#include "int8k_common.h"
#include "rows.h"

namespace int8k {
namespace {

__device__ __forceinline__ float load_any(const void* p, size_t i, int dtype) {
    switch (dtype) {
        case INT8K_DTYPE_F16: return __half2float(reinterpret_cast<const __half*>(p)[i]);
        case INT8K_DTYPE_BF16:
            return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
        default: return reinterpret_cast<const float*>(p)[i];
    }
}

// Rounds an fp32 value to the storage dtype and back (what a tensor of that
// dtype would hold), and stores it.
__device__ __forceinline__ float round_to(float v, int dtype) {
    switch (dtype) {
        case INT8K_DTYPE_F16: return __half2float(__float2half_rn(v));
        case INT8K_DTYPE_BF16: {
            // round to nearest even on the upper 16 bits (finite inputs)
            const uint32_t u = __float_as_uint(v);
            const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
            return __uint_as_float(r);
        }
        default: return v;
    }
}

__device__ __forceinline__ void store_any(void* p, size_t i, float v, int dtype) {
    switch (dtype) {
        case INT8K_DTYPE_F16: reinterpret_cast<__half*>(p)[i] = __float2half_rn(v); break;
        case INT8K_DTYPE_BF16:
            reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)(__float_as_uint(v) >> 16);
            break;
        default: reinterpret_cast<float*>(p)[i] = v;
    }
}

__device__ __forceinline__ int8_t quantize(float y, float s) {
    return (int8_t)(int)__builtin_rintf(fminf(fmaxf(y / s, -128.f), 127.f));
}

constexpr int kWaves = 4;
// Row kernels launch at most this many blocks (a launch must hold fewer than 2^32
// work-items) and stride over the remaining rows.
constexpr long long kMaxBlocks = 1LL << 20;
// The vectorised kernels stride over rows from a grid of at most this many
// blocks (about 8 resident blocks per CU of a 256-CU device, 4 rounds).
constexpr long long kVecBlocks = 8192;

template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = op(v, __shfl_xor(v, off));
    return v;
}

// One block of 4 waves per row.  Pass 1: mean; pass 2: centred sum of squares;
// pass 3: y and its absmax; pass 4: y again (bit-identical) and its codes.  The
// row is re-read from L2/L1 after the first pass.
__global__ __launch_bounds__(256) void layernorm_quant_kernel(
    const void* __restrict__ x, int dtype, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, int8_t* __restrict__ q, float* __restrict__ scales,
    void* __restrict__ y_out, long long rows, int cols) {
    __shared__ float red[kWaves];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    for (long long row = blockIdx.x; row < rows; row += gridDim.x) {  // < 2^32 work-items/launch
    const size_t base = (size_t)row * (size_t)cols;
    auto block_reduce = [&](float v, auto op) {
        v = wave_reduce(v, op);
        if (lane == 0) red[wave] = v;
        __syncthreads();
        float r = red[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) r = op(r, red[w]);
        __syncthreads();
        return r;
    };
    auto add = [](float a, float b) { return a + b; };
    auto mx = [](float a, float b) { return fmaxf(a, b); };

    float s = 0.f;
    for (int c = t; c < cols; c += 256) s += load_any(x, base + c, dtype);
    const float mean = block_reduce(s, add) / (float)cols;
    float v = 0.f;
    for (int c = t; c < cols; c += 256) {
        const float d = load_any(x, base + c, dtype) - mean;
        v = fmaf(d, d, v);
    }
    const float rstd = 1.f / sqrtf(block_reduce(v, add) / (float)cols + eps);
    auto ln = [&](int c) {
        float y = (load_any(x, base + c, dtype) - mean) * rstd;
        if (gamma) y *= gamma[c];
        if (beta) y += beta[c];
        return round_to(y, dtype);
    };
    float m = 0.f;
    for (int c = t; c < cols; c += 256) m = fmaxf(m, fabsf(ln(c)));
    const float sc = fmaxf(block_reduce(m, mx), 1e-8f) / 127.f;
    for (int c = t; c < cols; c += 256) {
        const float y = ln(c);
        q[base + c] = quantize(y, sc);
        if (y_out) store_any(y_out, base + c, y, dtype);
    }
    if (t == 0) scales[row] = sc;
    }
}

// One wave per source row (b, s, part, h) of Dh elements (grid-stride).
__global__ __launch_bounds__(256) void quant_heads_kernel(
    const void* __restrict__ x, int dtype, int8_t* __restrict__ q0, float* __restrict__ s0,
    int8_t* __restrict__ q1, float* __restrict__ s1, int8_t* __restrict__ q2,
    float* __restrict__ s2, long long rows, int S, int parts, int H, int Dh) {
    const int lane = threadIdx.x & 63;
    for (long long r = (long long)blockIdx.x * kWaves + (threadIdx.x >> 6); r < rows;
         r += (long long)gridDim.x * kWaves) {
        // r = ((b * S + s) * parts + p) * H + h
        const int h = (int)(r % H);
        const long long r1 = r / H;
        const int p = (int)(r1 % parts);
        const long long bs = r1 / parts;
        const long long b = bs / S, s = bs - b * S;
        const size_t src = (size_t)r * Dh;
        float m = 0.f;
        for (int c = lane; c < Dh; c += 64) m = fmaxf(m, fabsf(load_any(x, src + c, dtype)));
        m = wave_reduce(m, [](float a, float bb) { return fmaxf(a, bb); });
        const float sc = fmaxf(m, 1e-8f) / 127.f;
        int8_t* q = p == 0 ? q0 : (p == 1 ? q1 : q2);
        float* sp = p == 0 ? s0 : (p == 1 ? s1 : s2);
        const size_t drow = ((size_t)b * H + h) * S + s;  // [B, H, S] row of the part
        for (int c = lane; c < Dh; c += 64)
            q[drow * Dh + c] = quantize(load_any(x, src + c, dtype), sc);
        if (lane == 0) sp[drow] = sc;
    }
}

// ------------------------------------------------- vectorised paths (rows.h)

// Storage bits of y (already rounded to the dtype by round_to) for one chunk.
template <int DT>
__device__ __forceinline__ uint4 pack_chunk(const float (&y)[Vec<DT>::W]) {
    uint32_t d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (DT == INT8K_DTYPE_F32) {
            d[i] = __float_as_uint(y[i]);
        } else if constexpr (DT == INT8K_DTYPE_F16) {
            d[i] = (uint32_t)__half_as_ushort(__float2half_rn(y[2 * i])) |
                   ((uint32_t)__half_as_ushort(__float2half_rn(y[2 * i + 1])) << 16);
        } else {
            d[i] = (__float_as_uint(y[2 * i]) >> 16) | (__float_as_uint(y[2 * i + 1]) & 0xffff0000u);
        }
    }
    return make_uint4(d[0], d[1], d[2], d[3]);
}

// LayerNorm + per-token quantizer with the row in registers: 1 << lg lanes per
// row, NC 16-byte chunks per lane (chunk_slots).  One read of x; the passes of
// the one-element-per-lane kernel above become register passes.
template <int DT, int NC>
__global__ __launch_bounds__(256) void layernorm_quant_vec_kernel(
    const void* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    float eps, int8_t* __restrict__ q, float* __restrict__ scales, void* __restrict__ y_out,
    uint32_t rows, int lg, int nc) {
    constexpr int W = Vec<DT>::W;
    constexpr int NCMAX = chunk_slots<NC>();
    if (NC > 0) nc = NC;
    const int lane = threadIdx.x & 63;
    const uint32_t rpw = 64u >> lg;
    const uint32_t c0 = lane & ((1u << lg) - 1);
    const uint32_t cpr = (uint32_t)nc << lg;
    const int cols = (int)cpr * W;
    const float inv_cols = 1.f / (float)cols;
    const uint4* src = reinterpret_cast<const uint4*>(x);
    auto add = [](float a, float b) { return a + b; };
    const uint32_t nw = gridDim.x * 4;
    for (uint32_t rb = (blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw; rb < rows; rb += nw * rpw) {
        // rows past the end take the last row and store it again (the same bytes
        // its own lane stores): no divergent branch around loads or stores
        const uint32_t r = min(rb + (lane >> lg), rows - 1);
        uint4 w[NCMAX];
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < NCMAX; ++i) {
            if (NC > 0 || i < nc) {
                w[i] = src[(size_t)r * cpr + ((uint32_t)i << lg) + c0];
                float v[W];
                unpack_chunk<DT>(w[i], v);
#pragma unroll
                for (int e = 0; e < W; ++e) sum += v[e];
            }
        }
        const float mean = row_reduce(sum, lg, add) * inv_cols;
#pragma unroll
        for (int i = 0; i < NCMAX; ++i) reload_barrier(w[i]);
        float var = 0.f;
#pragma unroll
        for (int i = 0; i < NCMAX; ++i) {
            if (NC > 0 || i < nc) {
                float v[W];
                unpack_chunk<DT>(w[i], v);
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const float d = v[e] - mean;
                    var = fmaf(d, d, var);
                }
            }
        }
        const float rstd = 1.f / sqrtf(row_reduce(var, lg, add) * inv_cols + eps);
#pragma unroll
        for (int i = 0; i < NCMAX; ++i) reload_barrier(w[i]);
        // y, rounded to the dtype, replaces x in the chunk registers (its storage
        // bits: unpacking them gives the rounded values back exactly).  gamma and
        // beta are re-read per row (cache hits) instead of being hoisted out of
        // the row loop into registers.
        const float* g = gamma;
        const float* bt = beta;
        asm volatile("" : "+s"(g), "+s"(bt));
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < NCMAX; ++i) {
            if (NC > 0 || i < nc) {
                float y[W];
                unpack_chunk<DT>(w[i], y);
                const int col0 = (int)((((uint32_t)i << lg) + c0) * W);
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    float t = (y[e] - mean) * rstd;
                    if (g) t *= g[col0 + e];
                    if (bt) t += bt[col0 + e];
                    y[e] = round_to(t, DT);
                    m = fmaxf(m, fabsf(y[e]));
                }
                w[i] = pack_chunk<DT>(y);
            }
        }
        const float sc = fmaxf(row_reduce(m, lg, [](float a, float b) { return fmaxf(a, b); }),
                               1e-8f) / 127.f;
        const float inv = 1.f / sc;
#pragma unroll
        for (int i = 0; i < NCMAX; ++i) {
            if (NC > 0 || i < nc) {
                float y[W];
                unpack_chunk<DT>(w[i], y);
                const size_t chunk = (size_t)r * cpr + ((uint32_t)i << lg) + c0;
                store_codes<W>(y, sc, inv, q + chunk * W);
                if (y_out) reinterpret_cast<uint4*>(y_out)[chunk] = w[i];
            }
        }
        if (c0 == 0) scales[r] = sc;
    }
}

// Split-heads + per-token quantizer: source row ((b S + s) parts + p) H + h of
// Dh elements, 1 << lg lanes per row, one 16-byte chunk per lane.  Rows are
// walked in destination order k = ((p B + b) H + h) S + s, so the rows of a
// wave are consecutive tokens of one head: its codes and scales go out as one
// contiguous run (not as 64-byte pieces of H different heads), while each row
// is still read as one full source row.  Each wave takes U row groups of its
// grid stride at a time (U loads per lane in flight).
template <int DT, int U>
__global__ __launch_bounds__(256) void quant_heads_vec_kernel(
    const void* __restrict__ x, int8_t* __restrict__ q0, float* __restrict__ s0,
    int8_t* __restrict__ q1, float* __restrict__ s1, int8_t* __restrict__ q2,
    float* __restrict__ s2, uint32_t rows, uint32_t S, uint32_t parts, uint32_t H, int lg) {
    constexpr int W = Vec<DT>::W;
    const int lane = threadIdx.x & 63;
    const uint32_t rpw = 64u >> lg;
    const uint32_t c0 = lane & ((1u << lg) - 1);
    const int Dh = (1 << lg) * W;
    const uint4* src = reinterpret_cast<const uint4*>(x);
    const uint32_t stride = gridDim.x * 4 * rpw;
    const uint32_t part_rows = rows / parts;  // B H S rows per part
    for (uint32_t kb = (blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw; kb < rows; kb += U * stride) {
        uint4 w[U];
        uint32_t drow[U], pp[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // rows past the end take the last row: they load, quantize and store
            // it again, the same bytes its own lane stores.  No divergent branch
            // around the loads or the stores, which keeps them all in flight.
            const uint32_t k = min(kb + u * stride + (lane >> lg), rows - 1);
            pp[u] = k / part_rows;
            drow[u] = k - pp[u] * part_rows;  // (b H + h) S + s
            const uint32_t bh = drow[u] / S, s = drow[u] - bh * S;
            const uint32_t b = bh / H, h = bh - b * H;
            const uint32_t r = ((b * S + s) * parts + pp[u]) * H + h;
            w[u] = src[((size_t)r << lg) + c0];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float v[W];
            unpack_chunk<DT>(w[u], v);
            float m = 0.f;
#pragma unroll
            for (int e = 0; e < W; ++e) m = fmaxf(m, fabsf(v[e]));
            m = row_reduce(m, lg, [](float a, float b) { return fmaxf(a, b); });
            const float sc = fmaxf(m, 1e-8f) / 127.f;
            const float inv = 1.f / sc;
            int8_t* q = pp[u] == 0 ? q0 : (pp[u] == 1 ? q1 : q2);
            float* sp = pp[u] == 0 ? s0 : (pp[u] == 1 ? s1 : s2);
            store_codes<W>(v, sc, inv, q + (size_t)drow[u] * Dh + (size_t)c0 * W);
            if (c0 == 0) sp[drow[u]] = sc;
        }
    }
}

}  // namespace
}  // namespace int8k

using namespace int8k;

extern "C" int int8k_layernorm_quantize_per_token(const void* x, int dtype, const float* gamma,
                                                  const float* beta, float eps, int8_t* q,
                                                  float* scales, void* y_out, long long rows,
                                                  int cols, void* stream) {
    clear_last_error();
    if (!x || !q || !scales || rows < 0 || cols <= 0 || !(eps >= 0.f))
        return INT8K_ERR_INVALID_ARGUMENT;
    if (dtype != INT8K_DTYPE_F16 && dtype != INT8K_DTYPE_BF16 && dtype != INT8K_DTYPE_F32)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (rows == 0) return INT8K_OK;
    hipStream_t st = as_stream(stream);
    const RowShape sh = row_shape(cols, dtype);
    const int w = dtype == INT8K_DTYPE_F32 ? 4 : 8;
    if (sh.ok && rows < (1LL << 31) && aligned_to(x, 16) && aligned_to(q, w) &&
        (!y_out || aligned_to(y_out, 16))) {
        const long long waves = ceil_div(rows, 64 >> sh.lg);
        const unsigned blocks = (unsigned)std::min(ceil_div(waves, 4), kVecBlocks);
        with_dtype(dtype, [&](auto dt) {
            with_chunks(sh.nc, [&](auto ncc) {
                layernorm_quant_vec_kernel<decltype(dt)::value, decltype(ncc)::value>
                    <<<blocks, 256, 0, st>>>(x, gamma, beta, eps, q, scales, y_out,
                                             (uint32_t)rows, sh.lg, sh.nc);
            });
        });
        return check_launch("layernorm_quant_vec_kernel");
    }
    layernorm_quant_kernel<<<(unsigned)std::min(rows, kMaxBlocks), 256, 0, st>>>(
        x, dtype, gamma, beta, eps, q, scales, y_out, rows, cols);
    return check_launch("layernorm_quant_kernel");
}

extern "C" int int8k_quantize_heads(const void* x, int dtype, int parts, int8_t* q0, float* s0,
                                    int8_t* q1, float* s1, int8_t* q2, float* s2, int B, int S,
                                    int H, int head_dim, void* stream) {
    clear_last_error();
    if (!x || parts < 1 || parts > 3 || B <= 0 || S <= 0 || H <= 0 || head_dim <= 0)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (dtype != INT8K_DTYPE_F16 && dtype != INT8K_DTYPE_BF16 && dtype != INT8K_DTYPE_F32)
        return INT8K_ERR_INVALID_ARGUMENT;
    int8_t* qs[3] = {q0, q1, q2};
    float* ss[3] = {s0, s1, s2};
    for (int p = 0; p < parts; ++p)
        if (!qs[p] || !ss[p]) return INT8K_ERR_INVALID_ARGUMENT;
    const long long rows = (long long)B * S * parts * H;
    hipStream_t st = as_stream(stream);
    const RowShape sh = row_shape(head_dim, dtype);
    const int w = dtype == INT8K_DTYPE_F32 ? 4 : 8;
    bool vec = sh.ok && sh.nc == 1 && rows < (1LL << 31) && aligned_to(x, 16);
    for (int p = 0; p < parts; ++p) vec = vec && aligned_to(qs[p], w);
    if (vec) {
        constexpr int U = 4;
        const long long waves = ceil_div(rows, 64 >> sh.lg);
        const unsigned blocks = (unsigned)std::min(ceil_div(waves, 4 * U), kVecBlocks);
        with_dtype(dtype, [&](auto dt) {
            quant_heads_vec_kernel<decltype(dt)::value, U><<<blocks, 256, 0, st>>>(
                x, q0, s0, q1, s1, q2, s2, (uint32_t)rows, (uint32_t)S, (uint32_t)parts,
                (uint32_t)H, sh.lg);
        });
        return check_launch("quant_heads_vec_kernel");
    }
    quant_heads_kernel<<<(unsigned)std::min(ceil_div(rows, kWaves), kMaxBlocks), 256, 0, st>>>(
        x, dtype, q0, s0, q1, s1, q2, s2, rows, S, parts, H, head_dim);
    return check_launch("quant_heads_kernel");
}
