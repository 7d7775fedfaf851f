// int8k_common.h — shared host/device helpers for the gfx950 INT8 kernels.
//
// Internal header: only the .hip translation units of libint8k include it.
// Everything here is written for CDNA4 (wave64, DPP, v_dot4, MFMA); there is
// no other target.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include <atomic>

#include "int8k.h"

namespace int8k {

// ---------------------------------------------------------------- host side

// Records the text of a failing HIP call for int8k_last_error().
void set_last_error(const char* what, hipError_t err);
// Records a message of this library's own for int8k_last_error().
void set_last_error_text(const char* text);
void clear_last_error();

// Checks the launch that was just enqueued on this thread.
inline int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_last_error(what, err);
        return INT8K_ERR_HIP;
    }
    return INT8K_OK;
}

inline bool aligned_to(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
inline long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }

// Workspace sub-allocations are carved at this granularity.
constexpr size_t kWorkspaceAlign = 256;

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Set-up done once per device: hipFuncSetAttribute (the > 64 KiB dynamic LDS
// limit) applies to the current device, so a process driving several GPUs
// configures each.  Devices 0..63 are tracked (others run the set-up on every
// call); two threads racing on a device only repeat the idempotent set-up, and
// a failed set-up is tried again on the next call.
class PerDeviceOnce {
    std::atomic<uint64_t> done_{0};

public:
    template <typename F>
    int run(F&& setup) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return setup();
        const uint64_t bit = 1ull << dev;
        if (done_.load(std::memory_order_acquire) & bit) return INT8K_OK;
        const int st = setup();
        if (st == INT8K_OK) done_.fetch_or(bit, std::memory_order_release);
        return st;
    }
};

// -------------------------------------------------------------- device side

constexpr float kLog2e = 1.4426950408889634f;

// 2^x on the transcendental unit (v_exp_f32).  exp2(-inf) = 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane moves inside a row of 16 lanes (DPP, no LDS traffic).
// quad_perm [1,0,3,2]: lane ^ 1
__device__ __forceinline__ int dpp_xor1(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
}
// quad_perm [2,3,0,1]: lane ^ 2
__device__ __forceinline__ int dpp_xor2(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
}
// row_half_mirror: lane i of each 8-lane half-row reads lane 7-i.
__device__ __forceinline__ int dpp_half_mirror(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
}

// row_mirror: lane i of each 16-lane row reads lane 15-i.
__device__ __forceinline__ int dpp_row_mirror(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
}

// Sum over each aligned group of 4 lanes; every lane of the group gets it.
__device__ __forceinline__ int group4_sum(int v) {
    v += dpp_xor1(v);
    v += dpp_xor2(v);
    return v;
}
// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ __forceinline__ int group8_sum(int v) {
    v = group4_sum(v);
    v += dpp_half_mirror(v);
    return v;
}

// x combined with the value of lane ^ 32: v_permlane32_swap exchanges the two
// 32-lane halves on the VALU (no LDS round trip as with ds_bpermute); the
// pair it returns holds x of both lanes in either order.
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Signed byte i (0..3) of a packed dword as fp32 (one SDWA v_cvt_f32_i32).
template <int I>
__device__ __forceinline__ float sbyte_to_f32(int w) {
    return static_cast<float>(static_cast<int8_t>((w >> (8 * I)) & 0xff));
}

// fp32 -> fp16 bits, round to nearest even.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
    return __half_as_ushort(__float2half_rn(x));
}

// fp32 -> fp16 (round to nearest even) of x as an fp32 number.  clang folds
// half(a * b) into v_fma_mixlo_f16, which rounds the exact product to fp16 in
// one step; PyTorch's (q.float() * s).half() rounds it to fp32 first, and the
// two differ when that first rounding lands on an fp16 tie.  The empty asm
// pins x as the fp32 value, for outputs that must match bit for bit (not
// volatile: a volatile asm would also keep loads from being merged or moved
// across it).
__device__ __forceinline__ __half f16_of_f32(float x) {
    asm("" : "+v"(x));
    return __float2half_rn(x);
}

// Raw buffer resource over [base, base + bytes): loads at offsets past the end
// return zero, so tiles that overhang a matrix need no clamped addresses.  The
// arguments must be the same for the whole wave (they go to scalar registers).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buffer(const void* base, uint32_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint64_t ub =
        (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)))
         << 32) |
        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(ub), 0,
                                             __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Byte J of two dwords whose bytes were XORed with 0x80 (int8 -> biased
// uint8), as a packed pair of fp16 integers {lo: byte J of w0, hi: of w1}.
// 0x6400 | u is the fp16 value 1024 + u (exact for u < 1024), so one
// v_perm_b32, one OR and one v_pk_add_f16 convert two int8 values.
template <int J>
__device__ __forceinline__ uint32_t biased_bytes_to_f16x2(uint32_t w0x, uint32_t w1x) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    constexpr uint32_t sel = J | (0x0Cu << 8) | ((4u + J) << 16) | (0x0Cu << 24);
    const uint32_t u = __builtin_amdgcn_perm(w1x, w0x, sel) | 0x64006400u;
    h2 v = __builtin_bit_cast(h2, u);
    v = v + h2{(_Float16)-1152.0f, (_Float16)-1152.0f};
    return __builtin_bit_cast(uint32_t, v);
}

}  // namespace int8k
