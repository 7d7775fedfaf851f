// calib.hip — on-box ceilings for the roofline (built into libint8k_calib.so,
// used by bench.py only; not part of the C ABI of the kernels).
//
//   int8k_calib_stream_read : every lane streams 16-byte vectors through the
//       buffer (grid-stride), folds them with XOR and writes one word per
//       thread, so the HBM read bandwidth ceiling is bytes / time.
//   int8k_calib_copy        : plain 16-byte vector copy; its FETCH_SIZE /
//       WRITE_SIZE counters calibrate the PMC byte counts of other kernels.
//   int8k_calib_mfma_i8     : back-to-back v_mfma_i32_16x16x64_i8 on
//       independent accumulators, no memory traffic, giving the dense INT8
//       MFMA ceiling as 2*16*16*64 ops per instruction.
//   int8k_calib_mfma_i8_32_src : 16 independent v_mfma_i32_32x32x32_i8
//       accumulators per wave with operands loaded from a caller buffer, so
//       the sustained ceiling can be measured with the operand values a GEMM
//       sees (the MFMA rate this part sustains depends on the data: its power
//       draw sets the clock).
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void calib_stream_read_kernel(const int4* __restrict__ src,
                                                                size_t n_vec,
                                                                int* __restrict__ sink) {
    const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    int acc = 0;
    size_t i = tid;
    for (; i + 3 * stride < n_vec; i += 4 * stride) {
        const int4 a = src[i], b = src[i + stride], c = src[i + 2 * stride],
                   d = src[i + 3 * stride];
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^
               d.z ^ d.w;
    }
    for (; i < n_vec; i += stride) {
        const int4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    sink[tid] = acc;
}

typedef int v4i_t __attribute__((ext_vector_type(4)));

// Each wave streams its own contiguous chunk with 8 x 1 KiB loads in flight,
// non-temporal (the access pattern of the decode kernel's K/V stream).
__global__ __launch_bounds__(256) void calib_stream_chunk_nt_kernel(const v4i_t* __restrict__ src,
                                                                    size_t vec_per_wave,
                                                                    int* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    const size_t wave = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const v4i_t* p = src + wave * vec_per_wave + lane;
    int acc = 0;
    for (size_t i = 0; i + 8 * 64 <= vec_per_wave; i += 8 * 64) {
        v4i_t v[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = __builtin_nontemporal_load(p + i + t * 64);
#pragma unroll
        for (int t = 0; t < 8; ++t) acc ^= v[t].x ^ v[t].y ^ v[t].z ^ v[t].w;
    }
    sink[wave * 64 + lane] = acc;
}

__global__ __launch_bounds__(256) void calib_copy_kernel(const int4* __restrict__ src,
                                                         int4* __restrict__ dst, size_t n_vec) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_vec; i += stride)
        dst[i] = src[i];
}

__global__ __launch_bounds__(256) void calib_mfma_i8_kernel(int iters, int* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    v4i a = {lane, lane + 1, lane + 2, lane + 3};
    v4i b = {lane ^ 5, lane ^ 9, lane ^ 3, lane ^ 7};
    v4i c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c3, 0, 0, 0);
    }
    const v4i s = c0 + c1 + c2 + c3;
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s.x ^ s.y ^ s.z ^ s.w;
}

typedef int v16i_t __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void calib_mfma_i8_32_kernel(int iters, int* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    v4i a = {lane, lane + 1, lane + 2, lane + 3};
    v4i b = {lane ^ 5, lane ^ 9, lane ^ 3, lane ^ 7};
    v16i_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c3, 0, 0, 0);
    }
    const v16i_t s = c0 + c1 + c2 + c3;
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s[0] ^ s[5] ^ s[10] ^ s[15];
}

// One wave per SIMD at 256 blocks; operands a[4], b[4] per lane from src (8 KiB per block).
__global__ __launch_bounds__(256) void calib_mfma_i8_32_src_kernel(const v4i* __restrict__ src,
                                                                   int iters,
                                                                   int* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    v4i a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = src[(blockIdx.x * 8 + i) * 64 + lane];
        b[i] = src[(blockIdx.x * 8 + 4 + i) * 64 + lane];
    }
    v16i_t c[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) c[i] = v16i_t{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            c[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i & 3], b[i >> 2], c[i], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) s ^= c[i][0] ^ c[i][7] ^ c[i][15];
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

extern "C" int int8k_calib_stream_read(const void* buf, size_t bytes, int* sink, int blocks,
                                       void* stream) {
    calib_stream_read_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(
        (const int4*)buf, bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

// bytes must be a multiple of waves * 8 KiB; waves a multiple of 4.
extern "C" int int8k_calib_stream_chunk_nt(const void* buf, size_t bytes, int* sink, int waves,
                                           void* stream) {
    const size_t vec_per_wave = bytes / 16 / (size_t)waves;
    calib_stream_chunk_nt_kernel<<<waves / 4, 256, 0, (hipStream_t)stream>>>(
        (const v4i_t*)buf, vec_per_wave, sink);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

extern "C" int int8k_calib_copy(const void* src, void* dst, size_t bytes, int blocks,
                                void* stream) {
    calib_copy_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>((const int4*)src, (int4*)dst,
                                                               bytes / 16);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

// ops per launch = blocks * 4 waves * iters * 4 MFMAs * 65536
extern "C" int int8k_calib_mfma_i8_32(int blocks, int iters, int* sink, void* stream) {
    calib_mfma_i8_32_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(iters, sink);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

// ops per launch = blocks * 4 waves * iters * 16 MFMAs * 65536; src holds blocks * 8 KiB
extern "C" int int8k_calib_mfma_i8_32_src(const void* src, int blocks, int iters, int* sink,
                                          void* stream) {
    calib_mfma_i8_32_src_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>((const v4i*)src, iters,
                                                                         sink);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

// ops per launch = blocks * 4 waves * iters * 4 MFMAs * 32768
extern "C" int int8k_calib_mfma_i8(int blocks, int iters, int* sink, void* stream) {
    calib_mfma_i8_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(iters, sink);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}
