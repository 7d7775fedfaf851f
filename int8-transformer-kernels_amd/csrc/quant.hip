// quant.hip — quantization kernels: the reference's per-tensor quant utils and
// the per-token quantizer / INT8 KV-cache append that feed the attention paths.
//
//   per-tensor (kernels/quant_utils.cu:12-77):
//     amax = max|x| ; scale = max(amax, 1e-8) / 127 ; q = rn(clamp(x / scale))
//     dequant: half(q * scale)
//   The 1e-8 guard is deliberate: the reference kernel computes scale 0 on an
//   all-zero input and returns code -128 (kernels/quant_utils.cu:29-31,
//   39-40); every Python quantizer of the reference clamps amax to 1e-8.
//   per-token (validation/check_decode.py:42-47, tests/test_int8.py:47-63):
//     s_row = max(amax_row, 1e-8) / 127 ; q = rn(clamp(x / s_row, -128, 127))
//   Division (not a reciprocal multiply) and round-half-even keep the codes
//   bit-identical to torch's `(x.float() / s).round().clamp(-128, 127)`.
#include <algorithm>

#include "int8k_common.h"
#include "rows.h"

namespace int8k {
namespace {

__device__ __forceinline__ float load_elem(const void* p, size_t i, int dtype) {
    switch (dtype) {
        case INT8K_DTYPE_F16: return __half2float(reinterpret_cast<const __half*>(p)[i]);
        case INT8K_DTYPE_BF16: {
            const uint32_t b = reinterpret_cast<const uint16_t*>(p)[i];
            return __uint_as_float(b << 16);
        }
        default: return reinterpret_cast<const float*>(p)[i];
    }
}

__device__ __forceinline__ int8_t quant_div(float x, float s) {
    return (int8_t)(int)__builtin_rintf(fminf(fmaxf(x / s, -128.f), 127.f));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// ---------------------------------------------------------------- per tensor

__global__ void zero_f32_kernel(float* p) { *p = 0.f; }

__global__ __launch_bounds__(256) void amax_f16_kernel(const __half* __restrict__ x, size_t n,
                                                       float* __restrict__ amax) {
    __shared__ float red[4];
    float m = 0.f;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        m = fmaxf(m, fabsf(__half2float(x[i])));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        atomicMax(reinterpret_cast<int*>(amax), __float_as_int(m));  // m >= 0
    }
}

// Reads the tensor amax left in *scale by amax_f16_kernel; every block derives
// the same scale from it.
__global__ __launch_bounds__(256) void quant_tensor_f16_kernel(const __half* __restrict__ x,
                                                               int8_t* __restrict__ q, size_t n,
                                                               const float* __restrict__ amax) {
    const float s = fmaxf(*amax, 1e-8f) / 127.f;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        q[i] = quant_div(__half2float(x[i]), s);
}

__global__ void finalize_scale_kernel(float* scale) { *scale = fmaxf(*scale, 1e-8f) / 127.f; }

__global__ __launch_bounds__(256) void dequant_f16_kernel(const int8_t* __restrict__ q,
                                                          __half* __restrict__ y, size_t n,
                                                          float scale) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        y[i] = f16_of_f32((float)q[i] * scale);
}

// ---------------------------------------------------------------- per token

// General-shape path (row lengths the chunked kernel below cannot split, or
// unaligned pointers): one wave per row, one element per lane; amax pass, then
// the quantize pass (the row is re-read from cache).  `map_row(r)` maps source
// row r to its destination row, which is how the KV-cache append scatters new
// tokens into the cache.
struct RowMap {
    long long rows_per_group;  // source rows per (b,h) group (1 group: all rows)
    long long dst_group_stride;  // destination rows per group (cache capacity)
    long long dst_offset;      // first destination row inside a group
};

__device__ __forceinline__ long long map_row(long long r, const RowMap& m) {
    const long long g = r / m.rows_per_group, i = r - g * m.rows_per_group;
    return g * m.dst_group_stride + m.dst_offset + i;
}

__global__ __launch_bounds__(256) void quant_rows_kernel(const void* __restrict__ x, int dtype,
                                                         int8_t* __restrict__ q,
                                                         float* __restrict__ scales,
                                                         long long rows, int cols, RowMap map) {
    const int lane = threadIdx.x & 63;
    // grid-stride over rows: a launch holds fewer than 2^32 work-items
    for (long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows;
         r += (long long)gridDim.x * 4) {
        const size_t src = (size_t)r * cols;
        float m = 0.f;
        for (int c = lane; c < cols; c += 64) m = fmaxf(m, fabsf(load_elem(x, src + c, dtype)));
        m = wave_max(m);
        const float s = fmaxf(m, 1e-8f) / 127.f;
        const long long d = map_row(r, map);
        int8_t* qr = q + (size_t)d * cols;
        for (int c = lane; c < cols; c += 64) qr[c] = quant_div(load_elem(x, src + c, dtype), s);
        if (lane == 0) scales[d] = s;
    }
}

// Destination of source row r for the vectorised kernel: RowMap with 32-bit
// row arithmetic (the vectorised path requires fewer than 2^31 source rows).
struct RowDst {
    int8_t* q;
    float* scales;
    int cols;
    uint32_t rows_per_group;
    long long dst_group_stride, dst_offset;
    __device__ __forceinline__ void operator()(uint32_t r, int8_t*& qrow, float*& sp) const {
        const uint32_t g = r / rows_per_group, i = r - g * rows_per_group;
        const long long d = (long long)g * dst_group_stride + dst_offset + i;
        qrow = q + (size_t)d * cols;
        sp = scales + d;
    }
};

// Vectorised per-token quantizer (one 16-byte chunk per lane, see rows.h): the
// row is loaded once, kept in registers for the quantize step, and written as
// 4- or 8-byte code groups.  NC chunks per lane (chunk_slots).  Each wave takes
// U row groups of its grid stride at a time, so short rows still keep several
// loads per lane in flight.
template <int DT, int NC, int U>
__global__ __launch_bounds__(256) void quant_rows_vec_kernel(const void* __restrict__ x,
                                                             uint32_t rows, int lg, int nc,
                                                             RowDst dst) {
    constexpr int W = Vec<DT>::W;
    constexpr int SLOTS = chunk_slots<NC>();
    if (NC > 0) nc = NC;
    const int lane = threadIdx.x & 63;
    const uint32_t rpw = 64u >> lg;  // rows per wave
    const uint32_t c0 = lane & ((1u << lg) - 1);
    const uint32_t cpr = (uint32_t)nc << lg;  // chunks per row
    const uint4* src = reinterpret_cast<const uint4*>(x);
    const uint32_t stride = gridDim.x * 4 * rpw;  // rows between a wave's row groups
    for (uint32_t rb = (blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw; rb < rows; rb += U * stride) {
        uint4 w[U][SLOTS];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // rows past the end take the last row: they load, quantize and store
            // it again, the same bytes its own lane stores.  No divergent branch
            // around the loads or the stores, which keeps them all in flight.
            const uint32_t r = min(rb + u * stride + (lane >> lg), rows - 1);
#pragma unroll
            for (int i = 0; i < SLOTS; ++i)
                if (NC > 0 || i < nc) w[u][i] = src[(size_t)r * cpr + ((uint32_t)i << lg) + c0];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t r = min(rb + u * stride + (lane >> lg), rows - 1);
            float m = 0.f;
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                if (NC > 0 || i < nc) {
                    float v[W];
                    unpack_chunk<DT>(w[u][i], v);
#pragma unroll
                    for (int e = 0; e < W; ++e) m = fmaxf(m, fabsf(v[e]));
                }
            }
            m = row_reduce(m, lg, [](float a, float b) { return fmaxf(a, b); });
            const float s = fmaxf(m, 1e-8f) / 127.f;
            const float inv = 1.f / s;
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) reload_barrier(w[u][i]);
            int8_t* qrow;
            float* sp;
            dst(r, qrow, sp);
#pragma unroll
            for (int i = 0; i < SLOTS; ++i) {
                if (NC > 0 || i < nc) {
                    float v[W];
                    unpack_chunk<DT>(w[u][i], v);
                    store_codes<W>(v, s, inv, qrow + (size_t)(((uint32_t)i << lg) + c0) * W);
                }
            }
            if (c0 == 0) *sp = s;
        }
    }
}

// Per-token dequantization, the consumer side of the INT8 MLP / attention
// outputs: y[r, c] = T(float(q[r, c]) * s[r]) with T the rounding to the output
// dtype, and, with a residual, y = T(float(res[r, c]) + float(that)) — the
// values of PyTorch's `(q.float() * s[:, None]).to(dtype)` and of
// `res + that` in the residual's dtype.  The product is rounded to fp32 and
// then to the output dtype, and the add rounds again: FP contraction is off in
// these kernels (an FMA would round once for fp32) and f16_of_f32 keeps the
// fp16 conversion from fusing into the multiply.  16 codes per lane
// (cols % 16 == 0); the general path is one element per thread.
template <int DT>
__device__ __forceinline__ float round_dtype(float v) {
    if constexpr (DT == INT8K_DTYPE_F16) return __half2float(f16_of_f32(v));
    else if constexpr (DT == INT8K_DTYPE_BF16) {
        const uint32_t u = __float_as_uint(v);
        return __uint_as_float((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
    } else return v;
}

template <int DT>
__device__ __forceinline__ uint32_t dtype_bits16(float v) {  // v already rounded
    if constexpr (DT == INT8K_DTYPE_F16) return __half_as_ushort(__float2half_rn(v));
    else return __float_as_uint(v) >> 16;
}

template <int DT>
__device__ __forceinline__ float load_dtype(const void* p, size_t i) {
    if constexpr (DT == INT8K_DTYPE_F16)
        return __half2float(reinterpret_cast<const __half*>(p)[i]);
    else if constexpr (DT == INT8K_DTYPE_BF16)
        return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
    else return reinterpret_cast<const float*>(p)[i];
}

template <int DT>
__device__ __forceinline__ void store_dtype(void* p, size_t i, float v) {
    if constexpr (DT == INT8K_DTYPE_F32) reinterpret_cast<float*>(p)[i] = v;
    else reinterpret_cast<uint16_t*>(p)[i] = (uint16_t)dtype_bits16<DT>(v);
}

template <int DT, bool RES>
__global__ __launch_bounds__(256) void dequant_rows_vec_kernel(const int8_t* __restrict__ q,
                                                               const float* __restrict__ sc,
                                                               const void* __restrict__ res,
                                                               void* __restrict__ y,
                                                               uint32_t chunks, uint32_t cpr) {
#pragma clang fp contract(off)
    for (uint32_t g = blockIdx.x * 256 + threadIdx.x; g < chunks; g += gridDim.x * 256) {
        // 16 residual values: 2 (fp16/bf16) or 4 (fp32) 16-byte words
        constexpr int RW = DT == INT8K_DTYPE_F32 ? 4 : 2;
        uint32_t rd[4 * RW];
        if constexpr (RES) {
#pragma unroll
            for (int j = 0; j < RW; ++j) {
                const uint4 r = reinterpret_cast<const uint4*>(res)[(size_t)g * RW + j];
                rd[4 * j] = r.x, rd[4 * j + 1] = r.y, rd[4 * j + 2] = r.z, rd[4 * j + 3] = r.w;
            }
        }
        const uint4 w = reinterpret_cast<const uint4*>(q)[g];
        const float s = sc[g / cpr];
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
            v[i] = round_dtype<DT>((float)(int8_t)(wd[i >> 2] >> (8 * (i & 3))) * s);
        if constexpr (RES) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float r;
                if constexpr (DT == INT8K_DTYPE_F32) r = __uint_as_float(rd[i]);
                else if constexpr (DT == INT8K_DTYPE_F16)
                    r = __half2float(__ushort_as_half((unsigned short)(rd[i >> 1] >> (16 * (i & 1)))));
                else r = __uint_as_float((rd[i >> 1] >> (16 * (i & 1))) << 16);
                v[i] = round_dtype<DT>(r + v[i]);
            }
        }
        if constexpr (DT == INT8K_DTYPE_F32) {
            float4* o = reinterpret_cast<float4*>(y) + (size_t)g * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
        } else {
            uint32_t b[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                b[j] = dtype_bits16<DT>(v[2 * j]) | (dtype_bits16<DT>(v[2 * j + 1]) << 16);
            uint4* o = reinterpret_cast<uint4*>(y) + (size_t)g * 2;
            o[0] = make_uint4(b[0], b[1], b[2], b[3]);
            o[1] = make_uint4(b[4], b[5], b[6], b[7]);
        }
    }
}

template <int DT, bool RES>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const int8_t* __restrict__ q,
                                                           const float* __restrict__ sc,
                                                           const void* __restrict__ res,
                                                           void* __restrict__ y, size_t n,
                                                           int cols) {
#pragma clang fp contract(off)
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        float v = round_dtype<DT>((float)q[i] * sc[i / cols]);
        if constexpr (RES) v = round_dtype<DT>(load_dtype<DT>(res, i) + v);
        store_dtype<DT>(y, i, v);
    }
}

// Row kernels launch at most this many blocks and stride over the rest.
constexpr long long kMaxRowBlocks = 1LL << 20;
// The vectorised kernels stride over rows from a grid of at most this many
// blocks (about 8 resident blocks per CU of a 256-CU device, 4 rounds).
constexpr long long kVecRowBlocks = 8192;

int launch_quant_rows(const void* x, int dtype, int8_t* q, float* scales, long long rows,
                      int cols, const RowMap& map, hipStream_t stream) {
    if (rows <= 0) return INT8K_OK;
    const RowShape sh = row_shape(cols, dtype);
    const int w = dtype == INT8K_DTYPE_F32 ? 4 : 8;
    if (sh.ok && rows < (1LL << 31) && map.rows_per_group < (1LL << 31) && aligned_to(x, 16) &&
        aligned_to(q, w)) {
        const long long waves = ceil_div(rows, 64 >> sh.lg);
        const RowDst dst{q, scales, cols, (uint32_t)map.rows_per_group, map.dst_group_stride,
                         map.dst_offset};
        with_dtype(dtype, [&](auto dt) {
            with_chunks(sh.nc, [&](auto ncc) {
                constexpr int DT = decltype(dt)::value, NC = decltype(ncc)::value;
                constexpr int U = NC == 1 ? 4 : (NC == 2 ? 2 : 1);
                const unsigned blocks = (unsigned)std::min(ceil_div(waves, 4 * U), kVecRowBlocks);
                quant_rows_vec_kernel<DT, NC, U><<<blocks, 256, 0, stream>>>(
                    x, (uint32_t)rows, sh.lg, sh.nc, dst);
            });
        });
        return check_launch("quant_rows_vec_kernel");
    }
    const long long blocks = std::min((rows + 3) / 4, kMaxRowBlocks);
    quant_rows_kernel<<<(unsigned)blocks, 256, 0, stream>>>(x, dtype, q, scales, rows, cols, map);
    return check_launch("quant_rows_kernel");
}

inline int grid_for(long long n) {
    const long long b = (n + 255) / 256;
    return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace
}  // namespace int8k

using namespace int8k;

extern "C" int int8k_quantize_fp16_to_int8(const uint16_t* input, int8_t* output, float* d_scale,
                                           long long n, void* stream) {
    clear_last_error();
    if (!input || !output || !d_scale || n <= 0) return INT8K_ERR_INVALID_ARGUMENT;
    if (!aligned_to(input, 2) || !aligned_to(d_scale, 4)) return INT8K_ERR_MISALIGNED;
    hipStream_t s = as_stream(stream);
    const __half* x = reinterpret_cast<const __half*>(input);
    zero_f32_kernel<<<1, 1, 0, s>>>(d_scale);
    int st = check_launch("zero_f32_kernel");
    if (st != INT8K_OK) return st;
    amax_f16_kernel<<<grid_for(n), 256, 0, s>>>(x, (size_t)n, d_scale);
    if ((st = check_launch("amax_f16_kernel")) != INT8K_OK) return st;
    quant_tensor_f16_kernel<<<grid_for(n), 256, 0, s>>>(x, output, (size_t)n, d_scale);
    if ((st = check_launch("quant_tensor_f16_kernel")) != INT8K_OK) return st;
    finalize_scale_kernel<<<1, 1, 0, s>>>(d_scale);
    return check_launch("finalize_scale_kernel");
}

extern "C" int int8k_dequantize_int8_to_fp16(const int8_t* input, uint16_t* output, float scale,
                                             long long n, void* stream) {
    clear_last_error();
    if (!input || !output || n <= 0) return INT8K_ERR_INVALID_ARGUMENT;
    if (!aligned_to(output, 2)) return INT8K_ERR_MISALIGNED;
    dequant_f16_kernel<<<grid_for(n), 256, 0, as_stream(stream)>>>(
        input, reinterpret_cast<__half*>(output), (size_t)n, scale);
    return check_launch("dequant_f16_kernel");
}

extern "C" int int8k_quantize_per_token(const void* x, int dtype, int8_t* q, float* scales,
                                        long long rows, int cols, void* stream) {
    clear_last_error();
    if (!x || !q || !scales || rows <= 0 || cols <= 0) return INT8K_ERR_INVALID_ARGUMENT;
    if (dtype != INT8K_DTYPE_F16 && dtype != INT8K_DTYPE_BF16 && dtype != INT8K_DTYPE_F32)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (!aligned_to(x, dtype == INT8K_DTYPE_F32 ? 4 : 2) || !aligned_to(scales, 4))
        return INT8K_ERR_MISALIGNED;
    return launch_quant_rows(x, dtype, q, scales, rows, cols, RowMap{rows, rows, 0},
                             as_stream(stream));
}

extern "C" int int8k_kv_cache_append(const void* k_new, const void* v_new, int dtype,
                                     int8_t* K_cache, int8_t* V_cache, float* sK_cache,
                                     float* sV_cache, int BH, int n_new, int pos, int capacity,
                                     int head_dim, void* stream) {
    clear_last_error();
    if (!k_new || !v_new || !K_cache || !V_cache || !sK_cache || !sV_cache)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (BH <= 0 || n_new <= 0 || pos < 0 || capacity <= 0 || head_dim <= 0)
        return INT8K_ERR_INVALID_ARGUMENT;
    if ((long long)pos + n_new > capacity) return INT8K_ERR_INVALID_ARGUMENT;
    if (dtype != INT8K_DTYPE_F16 && dtype != INT8K_DTYPE_BF16 && dtype != INT8K_DTYPE_F32)
        return INT8K_ERR_INVALID_ARGUMENT;
    const size_t ea = dtype == INT8K_DTYPE_F32 ? 4 : 2;
    if (!aligned_to(k_new, ea) || !aligned_to(v_new, ea) || !aligned_to(sK_cache, 4) ||
        !aligned_to(sV_cache, 4))
        return INT8K_ERR_MISALIGNED;
    const RowMap map{n_new, capacity, pos};
    const long long rows = (long long)BH * n_new;
    hipStream_t s = as_stream(stream);
    int st = launch_quant_rows(k_new, dtype, K_cache, sK_cache, rows, head_dim, map, s);
    if (st != INT8K_OK) return st;
    return launch_quant_rows(v_new, dtype, V_cache, sV_cache, rows, head_dim, map, s);
}

extern "C" int int8k_dequantize_per_token(const int8_t* q, const float* scales, int dtype,
                                          const void* residual, void* y, long long rows,
                                          int cols, void* stream) {
    clear_last_error();
    if (!q || !scales || !y || rows < 0 || cols <= 0) return INT8K_ERR_INVALID_ARGUMENT;
    if (dtype != INT8K_DTYPE_F16 && dtype != INT8K_DTYPE_BF16 && dtype != INT8K_DTYPE_F32)
        return INT8K_ERR_INVALID_ARGUMENT;
    const size_t ea = dtype == INT8K_DTYPE_F32 ? 4 : 2;
    if (!aligned_to(scales, 4) || !aligned_to(y, ea) || (residual && !aligned_to(residual, ea)))
        return INT8K_ERR_MISALIGNED;
    if (rows == 0) return INT8K_OK;
    hipStream_t s = as_stream(stream);
    const size_t n = (size_t)rows * cols;
    const bool vec = cols % 16 == 0 && n / 16 < (1ULL << 32) && aligned_to(q, 16) &&
                     aligned_to(y, 16) && (!residual || aligned_to(residual, 16));
    with_dtype(dtype, [&](auto dt) {
        constexpr int DT = decltype(dt)::value;
        if (vec) {
            const uint32_t chunks = (uint32_t)(n / 16);
            const unsigned blocks = (unsigned)std::min<long long>(ceil_div(chunks, 256), 8192);
            if (residual)
                dequant_rows_vec_kernel<DT, true><<<blocks, 256, 0, s>>>(
                    q, scales, residual, y, chunks, (uint32_t)(cols / 16));
            else
                dequant_rows_vec_kernel<DT, false><<<blocks, 256, 0, s>>>(
                    q, scales, residual, y, chunks, (uint32_t)(cols / 16));
        } else {
            const unsigned blocks = (unsigned)std::min<long long>(ceil_div((long long)n, 256), 8192);
            if (residual)
                dequant_rows_kernel<DT, true><<<blocks, 256, 0, s>>>(q, scales, residual, y, n,
                                                                      cols);
            else
                dequant_rows_kernel<DT, false><<<blocks, 256, 0, s>>>(q, scales, residual, y, n,
                                                                       cols);
        }
    });
    return check_launch(vec ? "dequant_rows_vec_kernel" : "dequant_rows_kernel");
}
