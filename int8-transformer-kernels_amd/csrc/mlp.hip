// mlp.hip — INT8 two-GEMM MLP with dynamic per-token requantization (gfx950).
//
// Contract of the reference's int8_mlp_forward_impl dynamic path
// (kernels/int8_mlp.cu:999-1191) and its public launchers
// int8_mlp_forward / _per_channel / _per_channel_bias / _prepacked and
// transpose_int8_weights (kernels/int8_mlp.cu:1231-1314):
//
//   GEMM1   acc1 = x . W1                       (s8 x s8 -> exact s32)
//   epi1    v = (f32(acc1) * sx[t]) * sW1[n] (+ b1[n]);  v = GELU_tanh(v)
//           hidden = fp16(v);  rowmax_t = max_n |v|  (fp32, before rounding)
//   requant hq = rn(clamp(f32(hidden) * 127/max(rowmax,1e-8)));  sh[t] = max(rowmax,1e-8)/127
//   GEMM2   acc2 = hq . W2
//   epi2    o = (f32(acc2) * sh[t]) * sW2[n];  out16 = fp16(o);  rowmax / tensor max of |o|
//   quant   out = rn(clamp(f32(out16) * 127/amax)),  out_scale = amax/127 (per token or tensor)
//
// Kernels: gemm_i8_rq_kernel<EPI> (the MFMA core of gemm_i8.h whose epilogue
// finishes the per-token requantization itself: the tiles of a 256-row stripe
// exchange their row maxima through device-scope atomics and emit int8 codes,
// so neither the fp16 hidden nor the fp16 output reaches memory — the default
// wherever a GEMM runs 256 x 256 tiles), gemm_i8_kernel<EPI> (the same core with
// an fp16 epilogue: scales, bias, GELU, fp16 store and per-(tile, row) absmax
// partials), requant_rows_kernel (reduces the partials, requantizes a row; the
// path of the other tilings and of INT8K_MLP_SEPARATE_REQUANT),
// tensor_absmax_kernel and transpose_i8_kernel (weight packing to the
// K-contiguous [N][K] layout the MFMA operands want).
// gemm_i8_a16_kernel is GEMM2 reading the fp16 hidden and quantizing it per
// row on load (no requant pass, no int8 hidden in memory); same bytes, slower
// on MI355X, so it runs only when INT8K_MLP_GEMM2_FP16_HIDDEN=1.
//
// Few tokens (decode-time MLPs, T = B): 256 x 256 tiles leave most CUs idle
// (T = 128 gives 16 blocks for GEMM1 and 4 for GEMM2).  When a GEMM has fewer
// tiles than CUs it runs split-K instead: gemm_i8_splitk_kernel (128 x 128
// output tiles, the K range split over blocks, exact int32 partials) and
// splitk_epilogue_kernel<EPI> (sums the partials per row, then the same
// epilogue math as gemm_i8_kernel, writing the same fp16 output and absmax
// partials), so requant_rows_kernel and every result are the same on both
// paths.  Above 512 rows, a GEMM whose 256 x 256 grid has at most 128 tiles runs
// gemm_i8_mid_kernel<EPI> (128 x 128 tiles, two blocks per CU, the same
// epilogue), e.g. GEMM2 at T = 4096, d_model 1024.
#include <algorithm>
#include <cstdlib>

#include "gemm_i8.h"

namespace int8k {
namespace {

using namespace gemm;

enum EpiMode { EPI_I32 = 0, EPI_GELU_F16 = 1, EPI_F16 = 2 };

struct EpiParams {
    int32_t* c32;        // EPI_I32 output
    uint16_t* c16;       // fp16 output
    int ldc;
    const float* sa;     // per-row scale (stride sa_stride: 0 = scalar)
    int sa_stride;
    const float* sb;     // per-column scale
    int sb_stride;
    const float* bias;   // per-column bias or null
    float* pmax;         // [tiles_n][M] row absmax partials
};

// GELU, tanh form: 0.5 x (1 + tanh(u)) = x * sigmoid(2u), u = sqrt(2/pi)(x + 0.044715 x^3),
// as x / (1 + 2^y) with y = -2 log2(e) u = x (c0 + c1 x^2): four VALU ops, exp and rcp.
__device__ __forceinline__ float gelu_exponent(float x) {
    constexpr float c0 = (float)(-2.0 * 1.4426950408889634 * 0.7978845608028654);
    constexpr float c1 = (float)(-2.0 * 1.4426950408889634 * 0.7978845608028654 * 0.044715);
    return x * __builtin_fmaf(c1, x * x, c0);
}
__device__ __forceinline__ float gelu_tanh(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + fast_exp2(gelu_exponent(x)));
}

// Row scales, column scales and bias of a tile, parked in LDS after the main
// loop's stages: 3 x 256 floats.
constexpr int kEpiLdsBytes = LDS_BYTES + 3 * BM * 4;
static_assert(BM == kThreads && BN == kThreads, "one scale of each kind per thread");

// Epilogue value of accumulator element acc with row scale sa, column scale sb, bias b.
template <int EPI>
__device__ __forceinline__ float epi_value(int acc, float sa, float sb, float b) {
    float v = static_cast<float>(acc) * sa * sb;
    if constexpr (EPI == EPI_GELU_F16) v = gelu_tanh(v + b);
    return v;
}

// Row maxima of one 32-row block of a wave's sub-tile: rmax[r] holds the lane's
// max over its columns for row acc_row(r, lane).  The max over the 32 lanes
// that share those rows (one half of the wave) is taken stage by stage for
// all 16 rows: DPP inside each 16-lane row, then v_permlane16_swap across the
// two rows of the half (VALU only, no LDS round trip).  Lanes 0 and 32 then
// write the 16 values as four runs of 4 consecutive rows into `slot` (the
// block's rows of this wave's column half).
__device__ __forceinline__ void tile_rowmax(const float (&rmax)[16], int* slot, int lane) {
    int m[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) m[r] = __float_as_int(rmax[r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) m[r] = max(m[r], dpp_xor1(m[r]));
#pragma unroll
    for (int r = 0; r < 16; ++r) m[r] = max(m[r], dpp_xor2(m[r]));
#pragma unroll
    for (int r = 0; r < 16; ++r) m[r] = max(m[r], dpp_half_mirror(m[r]));
#pragma unroll
    for (int r = 0; r < 16; ++r) m[r] = max(m[r], dpp_row_mirror(m[r]));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const auto s = __builtin_amdgcn_permlane16_swap(m[r], m[r], false, false);
        m[r] = max((int)s[0], (int)s[1]);
    }
    if ((lane & 31) == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<int4*>(slot + q * 8 + (lane >> 5) * 4) =
                make_int4(m[4 * q], m[4 * q + 1], m[4 * q + 2], m[4 * q + 3]);
    }
}

// Interior tiles (every row and column in range, tile rows * ldc * 2 < 2^32): the
// fp16 tile goes out through a buffer resource at the tile's corner, so each
// store's address is the lane's fixed offset plus a uniform (scalar) one.
// Rows r, r+1 of a column sit in one lane and columns c, c+1 in lanes 2k,
// 2k+1: the lane converts its pair of rows into one word (v_cvt_pk_f16_f32),
// swaps it with the neighbour lane (DPP), and one byte permute leaves the
// even lane (r, c..c+1) and the odd lane (r+1, c..c+1) to store as one dword.
template <int EPI, int TM_ = TM, int TN_ = TN, int WM_ = WM, int WN_ = WN, int BM_ = BM>
__device__ __forceinline__ void epilogue_interior(const v16i (&acc)[TM_][TN_], const EpiParams& p,
                                                  int m0, int n0, int* rowmax, const float* esa,
                                                  const float* esb, const float* ebias) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const bool odd = lane & 1;
    const __amdgpu_buffer_rsrc_t out =
        make_buffer(p.c16 + (size_t)m0 * p.ldc + n0, (uint32_t)(BM_ * p.ldc * 2));
    const uint32_t voff =
        ((uint32_t)(wm * WM_ + (lane >> 5) * 4 + (odd ? 1 : 0)) * p.ldc + wn * WN_ + (lane & 30)) * 2;
    const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
    float sbv[TN_], biv[TN_];
#pragma unroll
    for (int j = 0; j < TN_; ++j) {
        sbv[j] = esb[wn * WN_ + j * 32 + (lane & 31)];
        biv[j] = ebias[wn * WN_ + j * 32 + (lane & 31)];
    }
#pragma unroll
    for (int i = 0; i < TM_; ++i) {
        // rows (r/4)*8 + (lane/32)*4 + r%4: four runs of 4 consecutive rows
        float sav[16], rmax[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 s4 =
                *reinterpret_cast<const float4*>(esa + wm * WM_ + i * 32 + q * 8 + (lane >> 5) * 4);
            sav[4 * q] = s4.x, sav[4 * q + 1] = s4.y, sav[4 * q + 2] = s4.z, sav[4 * q + 3] = s4.w;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) rmax[r] = 0.f;
        uint32_t words[TN_][8];  // packed fp16 pairs, stored once all column tiles are done
#pragma unroll
        for (int j = 0; j < TN_; ++j) {
            // stage by stage over the 16 elements, so one wave per SIMD has
            // independent work between the dependent steps of each element
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = static_cast<float>(acc[i][j][r]) * sav[r] * sbv[j];
            if constexpr (EPI == EPI_GELU_F16) {
                float e[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = v[r] + biv[j];
#pragma unroll
                for (int r = 0; r < 16; ++r) e[r] = gelu_exponent(v[r]);
#pragma unroll
                for (int r = 0; r < 16; ++r) e[r] = fast_exp2(e[r]);
#pragma unroll
                for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_rcpf(1.f + e[r]);
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = v[r] * e[r];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) rmax[r] = fmaxf(rmax[r], fabsf(v[r]));
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const h2 h = __builtin_convertvector((f2){v[r], v[r + 1]}, h2);
                const uint32_t own = __builtin_bit_cast(uint32_t, h);
                const uint32_t nb = __builtin_amdgcn_mov_dpp(own, 0xB1, 0xF, 0xF, true);
                words[j][r >> 1] = __builtin_amdgcn_perm(nb, own, sel);
            }
        }
        // row by row, the column tiles' stores of a row back to back: the 64-byte pieces
        // of each 128-byte line reach the cache together
#pragma unroll
        for (int r = 0; r < 16; r += 2)
#pragma unroll
            for (int j = 0; j < TN_; ++j) {
                const uint32_t soff = ((uint32_t)(i * 32 + (r >> 2) * 8 + (r & 3)) * p.ldc + j * 32) * 2;
                __builtin_amdgcn_raw_buffer_store_b32(words[j][r >> 1], out, voff, soff, 0);
            }
        tile_rowmax(rmax, rowmax + wn * BM_ + wm * WM_ + i * 32, lane);
    }
}

// Tiles on the matrix edge: the same values, element stores guarded by row < M
// and column < N, and the row maxima over in-range columns only.
template <int EPI, int TM_ = TM, int TN_ = TN, int WM_ = WM, int WN_ = WN, int BM_ = BM>
__device__ __forceinline__ void epilogue_edge(const v16i (&acc)[TM_][TN_], const EpiParams& p,
                                              int M, int N, int m0, int n0, int* rowmax,
                                              const float* esa, const float* esb,
                                              const float* ebias) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int rbase = m0 + wm * WM_;
    const int cbase = n0 + wn * WN_ + (lane & 31);
#pragma unroll
    for (int i = 0; i < TM_; ++i) {
        float rmax[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) rmax[r] = 0.f;
#pragma unroll
        for (int j = 0; j < TN_; ++j) {
            const int cl = wn * WN_ + j * 32 + (lane & 31);
            const bool cok = n0 + cl < N;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rl = wm * WM_ + i * 32 + acc_row(r, lane);
                const float v = epi_value<EPI>(acc[i][j][r], esa[rl], esb[cl], ebias[cl]);
                if (cok) rmax[r] = fmaxf(rmax[r], fabsf(v));
                const int row = rbase + i * 32 + acc_row(r, lane);
                if (row < M && cok) p.c16[(size_t)row * p.ldc + cbase + j * 32] = f32_to_f16_bits(v);
            }
        }
        tile_rowmax(rmax, rowmax + wn * BM_ + wm * WM_ + i * 32, lane);
    }
}

// The tile's epilogue after the main loop: fp16 stores and the per-(tile, row)
// absmax partial pmax[tn][row].  pre_sa/pre_sb/pre_b: this thread's row scale
// (row m0 + t), column scale and bias (column n0 + t), loaded before the main
// loop so it hides their latency.
template <int EPI, int TM_ = TM, int TN_ = TN, int WM_ = WM, int WN_ = WN, int BM_ = BM,
          int kScaleOff = LDS_BYTES>
__device__ __forceinline__ void epilogue_tile(const v16i (&acc)[TM_][TN_], const EpiParams& p,
                                              int M, int N, int m0, int n0, int tn, float pre_sa,
                                              float pre_sb, float pre_b, char* lds) {
    // Row absmax of this block's tile: rowmax[wn][row] from each column
    // half of the waves, combined below (values >= 0, so integer max on
    // the bit pattern orders them like floats).  The scale region lies
    // past the stages; the row maxima reuse stage 0, whose last reads
    // (operands past the end of K) are never used.  Square tiles of BM_
    // rows; threads t < BM_ hold row t's scale and column t's scale and bias.
    static_assert(BM_ <= kThreads && 2 * WM_ == BM_ && 2 * WN_ == BM_, "2 x 2 waves");
    int* rowmax = reinterpret_cast<int*>(lds);
    float* esa = reinterpret_cast<float*>(lds + kScaleOff);
    float* esb = esa + BM_;
    float* ebias = esb + BM_;
    const bool holder = BM_ == kThreads || (int)threadIdx.x < BM_;
    if (holder) {
        esa[threadIdx.x] = pre_sa;
        esb[threadIdx.x] = pre_sb;
        ebias[threadIdx.x] = pre_b;
    }
    __syncthreads();
    if (m0 + BM_ <= M && n0 + BM_ <= N && (size_t)BM_ * p.ldc * 2 < (1ull << 32))
        epilogue_interior<EPI, TM_, TN_, WM_, WN_, BM_>(acc, p, m0, n0, rowmax, esa, esb, ebias);
    else
        epilogue_edge<EPI, TM_, TN_, WM_, WN_, BM_>(acc, p, M, N, m0, n0, rowmax, esa, esb,
                                                     ebias);
    __syncthreads();
    const int row = m0 + threadIdx.x;
    if (holder && row < M)
        p.pmax[(size_t)tn * M + row] =
            __int_as_float(max(rowmax[threadIdx.x], rowmax[BM_ + threadIdx.x]));
}

// BKN: Bt is B stored [K][N] (ldb = its row stride), read without a transpose.
template <int EPI, bool BKN = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_i8_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ Bt, int M, int N, int K, int lda,
    int ldb, int tiles_m, int tiles_n, EpiParams p) {
    extern __shared__ __align__(16) char lds[];
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // The epilogue's scales and bias for this tile, loaded before the main loop
    // (clamped indices, so unconditional) so the loop hides their latency.
    float pre_sa = 0.f, pre_sb = 0.f, pre_b = 0.f;
    if constexpr (EPI != EPI_I32) {
        const int t = threadIdx.x;
        pre_sa = p.sa[(size_t)min(m0 + t, M - 1) * p.sa_stride];
        pre_sb = p.sb[(size_t)min(n0 + t, N - 1) * p.sb_stride];
        if (p.bias != nullptr) pre_b = p.bias[min(n0 + t, N - 1)];
    }
    v16i acc[TM][TN];
    // interior tiles take the unmasked operand path
    if (m0 + BM <= M && n0 + BN <= N && K % BK == 0)
        mainloop<false, false, BKN>(acc, A, Bt, M, N, K, lda, ldb, m0, n0, lds);
    else
        mainloop<true, false, BKN>(acc, A, Bt, M, N, K, lda, ldb, m0, n0, lds);

    if constexpr (EPI == EPI_I32) {
        const int lane = threadIdx.x & 63;
        const int wave = threadIdx.x >> 6;
        const int wm = wave >> 1, wn = wave & 1;
        const int rbase = m0 + wm * WM;
        const int cbase = n0 + wn * WN + (lane & 31);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = cbase + j * 32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = rbase + i * 32 + acc_row(r, lane);
                    if (row < M && col < N) p.c32[(size_t)row * p.ldc + col] = acc[i][j][r];
                }
            }
        return;
    } else {
        epilogue_tile<EPI>(acc, p, M, N, m0, n0, tn, pre_sa, pre_sb, pre_b, lds);
    }
}

// ------------------------------------------------------------ requant fused into the GEMM
// gemm_i8_rq_kernel<EPI>: gemm_i8_kernel whose epilogue also finishes the
// per-token requantization, so the fp16 rows never reach memory and no
// requant pass runs.  The row max that a code needs spans every column tile
// of the row's 256-row stripe, so the tiles of a stripe exchange it:
//   1. each tile computes v (scales, bias, GELU) and fp16(v) from its live
//      accumulators, keeps the fp16 pairs in registers and reduces the row
//      maxima of |v| over its 256 columns (fp32, before rounding);
//   2. it folds them into amax[row] (device-scope atomic max on the float
//      bits: |v| >= 0 orders like the integers) and, once those atomics have
//      completed, adds one to arrived[stripe];
//   3. one lane waits until arrived[stripe] counts every tile of the stripe,
//      reading the counter and then amax[row] with device-scope atomic loads
//      (they bypass the XCD's L2, so no cache flush is needed);
//   4. code = rint(clamp(f32(fp16(v)) * (127 / max(amax, 1e-8)))), the
//      expression of requant_rows_kernel, so the codes are that pass's codes
//      byte for byte; the stripe's column-0 tile writes the row scales
//      max(amax, 1e-8) / 127.
// The wait needs every tile of a stripe resident at once.  Blocks map to
// tiles in groups of stripes; inside a group each XCD (block id % 8) takes a
// panel of stripes x columns and walks it stripe by stripe, so a stripe's
// tiles come right after the tiles of earlier stripes in every XCD's
// dispatch order: with blocks dispatched in id order, a stripe is waited on
// only once all its tiles are resident or done.  The host takes this path
// only when a stripe has at most kRqMaxStripeTiles tiles (half the CUs).  The
// wait is bounded in time nevertheless (every wave exits); a wait that gives
// up counts in g_rq_timeouts (int8k_mlp_sync_timeouts) and the tile then
// uses the maxima that have arrived.
constexpr int kRqMaxStripeTiles = 128;
constexpr unsigned long long kRqWaitTicks = 1ull << 26;  // s_memrealtime (100 MHz): ~0.67 s

__device__ unsigned int g_rq_timeouts;

struct RqParams {
    int8_t* q;           // codes [M][ldq]
    int ldq;
    float* scales;       // [M] row scale max(amax, 1e-8) / 127
    uint32_t* amax;      // [M] max |v| of the row as float bits; zero before the launch
    uint32_t* arrived;   // [tiles_m] tiles of the stripe that published; zero before the launch
    int gs;              // stripes per group
    int xm, xn;          // XCD panel grid of a group (xm * xn == 8); xn == 0: stripe-major order
};

// Block id -> (stripe, column tile); see the dispatch-order note above.
__device__ __forceinline__ void rq_tile_coords(int bid, int tiles_m, int tiles_n,
                                               const RqParams& rq, int& tm, int& tn) {
    const int per_group = rq.gs * tiles_n;
    const int g = bid / per_group, b = bid - g * per_group;
    const int s0 = g * rq.gs;
    if (rq.xn > 0 && s0 + rq.gs <= tiles_m) {
        const int x = b % kNumXcd, l = b / kNumXcd;
        const int pn = tiles_n / rq.xn, pm = rq.gs / rq.xm;
        tm = s0 + (x % rq.xm) * pm + l / pn;
        tn = (x / rq.xm) * pn + l % pn;
    } else {
        tm = s0 + b / tiles_n;
        tn = b % tiles_n;
    }
}

// Codes of the two fp16 values of `pair` with inverse scale inv, each as the low
// byte of a float's bits: fl(h * inv) (one v_fma_mix rounding, the pass's
// multiply; the sign of a zero product does not reach the code), clamped to
// [-128, 127] when CLAMP, plus 1.5 * 2^23, which rounds half to even onto the
// integer grid as rint does in requant_rows_kernel.  Without CLAMP the caller
// guarantees |h * inv| < 127.5: every row max of the tile in [2^-14, 65504],
// so h = fp16(v) <= amax (1 + 2^-11) + 2^-25 is finite.
template <bool CLAMP>
__device__ __forceinline__ uint32_t rq_codes4(uint32_t p01, uint32_t p23, float inv) {
#pragma clang fp contract(off)
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 a = __builtin_bit_cast(h2, p01), b = __builtin_bit_cast(h2, p23);
    float f[4] = {__builtin_fmaf((float)a.x, inv, 0.0f), __builtin_fmaf((float)a.y, inv, 0.0f),
                  __builtin_fmaf((float)b.x, inv, 0.0f), __builtin_fmaf((float)b.y, inv, 0.0f)};
    uint32_t c[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if constexpr (CLAMP) f[k] = fminf(fmaxf(f[k], -128.f), 127.f);
        c[k] = __float_as_uint(f[k] + 12582912.0f);
    }
    return __builtin_amdgcn_perm(c[1], c[0], 0x0c0c0400u) |
           __builtin_amdgcn_perm(c[3], c[2], 0x04000c0cu);
}

// The fp16 tile waits in LDS (the operand stages are free after the main loop),
// row-major with rows padded to kRqHStride bytes; the row maxima of the two
// column halves of the waves follow it.
constexpr int kRqHStride = 2 * BN + 8;
constexpr int kRqRowmaxOff = BM * kRqHStride;
static_assert(kRqRowmaxOff + 2 * BM * 4 <= LDS_BYTES, "fp16 tile and row maxima fit the stages");

// Step 4 of the fused epilogue: each thread turns 16-column pieces of whole rows
// of the staged fp16 tile into 16 codes and stores them as 16 bytes, so a
// wave's store covers 8 full 128-byte lines.  einv: 127 / amax per tile row.
template <bool CLAMP>
__device__ __forceinline__ void rq_store_codes(const char* lds, const float* einv,
                                               const RqParams& rq, int M, int N, int m0, int n0) {
    const int t = threadIdx.x;
    constexpr int kPieces = BM * BN / 16 / kThreads;  // 16 per thread; 16 threads per row
    const int g = t & 15;
    const bool vec = (reinterpret_cast<uintptr_t>(rq.q) & 15) == 0 && (rq.ldq & 15) == 0;
    const bool interior = vec && m0 + BM <= M && n0 + BN <= N;
#pragma unroll 4
    for (int k = 0; k < kPieces; ++k) {
        const int row = (t >> 4) + 16 * k;
        const float inv = einv[row];
        const uint2* src = reinterpret_cast<const uint2*>(lds + row * kRqHStride + g * 32);
        const uint2 h0 = src[0], h1 = src[1], h2v = src[2], h3 = src[3];
        const uint4 c = make_uint4(rq_codes4<CLAMP>(h0.x, h0.y, inv),
                                   rq_codes4<CLAMP>(h1.x, h1.y, inv),
                                   rq_codes4<CLAMP>(h2v.x, h2v.y, inv),
                                   rq_codes4<CLAMP>(h3.x, h3.y, inv));
        int8_t* dst = rq.q + (size_t)(m0 + row) * rq.ldq + n0 + g * 16;
        if (interior) {
            *reinterpret_cast<uint4*>(dst) = c;
        } else if (m0 + row < M && n0 + g * 16 < N) {
            // N is a multiple of 16: a piece is wholly in or out
            uint32_t* d4 = reinterpret_cast<uint32_t*>(dst);
            d4[0] = c.x, d4[1] = c.y, d4[2] = c.z, d4[3] = c.w;
        }
    }
}

// The fused epilogue on the swapped accumulator layout (mainloop<*, true>): lane
// l holds row l % 32 of each 32-row block i and, for each column tile j, the
// 16 columns (r/4)*8 + (l/32)*4 + r%4.  v and its row maxima as in
// epilogue_interior; fp16(v) goes to LDS right away, so no value is held in
// registers across the wait.
template <int EPI>
__device__ __forceinline__ void epilogue_rq(const v16i (&acc)[TM][TN], const RqParams& rq,
                                            int M, int N, int m0, int n0, int tm, int tn,
                                            int tiles_n, float pre_sa, float pre_sb,
                                            float pre_b, char* lds) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5;
    int* rowmax = reinterpret_cast<int*>(lds + kRqRowmaxOff);  // [2][BM]
    float* esa = reinterpret_cast<float*>(lds + LDS_BYTES);
    float* esb = esa + BM;
    float* ebias = esb + BM;
    esa[t] = pre_sa;
    esb[t] = pre_sb;
    ebias[t] = pre_b;
    __syncthreads();
    // 1. values, the row max of |v| (columns past N excluded), fp16 pairs to LDS
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int rl = wm * WM + i * 32 + (lane & 31);
        const float sa = esa[rl];
        char* hrow = lds + rl * kRqHStride;
        float rmax = 0.f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int c0 = wn * WN + j * 32 + half * 4;  // + q * 8 + k
            float v[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 sb4 = *reinterpret_cast<const float4*>(esb + c0 + q * 8);
                v[4 * q] = static_cast<float>(acc[i][j][4 * q]) * sa * sb4.x;
                v[4 * q + 1] = static_cast<float>(acc[i][j][4 * q + 1]) * sa * sb4.y;
                v[4 * q + 2] = static_cast<float>(acc[i][j][4 * q + 2]) * sa * sb4.z;
                v[4 * q + 3] = static_cast<float>(acc[i][j][4 * q + 3]) * sa * sb4.w;
            }
            if constexpr (EPI == EPI_GELU_F16) {
                float e[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 b4 = *reinterpret_cast<const float4*>(ebias + c0 + q * 8);
                    v[4 * q] = v[4 * q] + b4.x;
                    v[4 * q + 1] = v[4 * q + 1] + b4.y;
                    v[4 * q + 2] = v[4 * q + 2] + b4.z;
                    v[4 * q + 3] = v[4 * q + 3] + b4.w;
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) e[r] = gelu_exponent(v[r]);
#pragma unroll
                for (int r = 0; r < 16; ++r) e[r] = fast_exp2(e[r]);
#pragma unroll
                for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_rcpf(1.f + e[r]);
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = v[r] * e[r];
            }
            if (n0 + BN <= N) {
#pragma unroll
                for (int r = 0; r < 16; ++r) rmax = fmaxf(rmax, fabsf(v[r]));
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (n0 + c0 + (r >> 2) * 8 + (r & 3) < N) rmax = fmaxf(rmax, fabsf(v[r]));
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t p01 = __builtin_bit_cast(
                    uint32_t, __builtin_convertvector((f2){v[4 * q], v[4 * q + 1]}, h2));
                const uint32_t p23 = __builtin_bit_cast(
                    uint32_t, __builtin_convertvector((f2){v[4 * q + 2], v[4 * q + 3]}, h2));
                *reinterpret_cast<uint2*>(hrow + (c0 + q * 8) * 2) = make_uint2(p01, p23);
            }
        }
        // lanes l and l ^ 32 hold the same row
        const auto s = __builtin_amdgcn_permlane32_swap(__float_as_int(rmax), __float_as_int(rmax),
                                                        false, false);
        const int m = max((int)s[0], (int)s[1]);
        if (half == 0) rowmax[wn * BM + rl] = m;
    }
    __syncthreads();
    // 2. publish the tile's row maxima, then its arrival
    const int row_t = m0 + t;
    if (row_t < M) {
        const uint32_t m = (uint32_t)max(rowmax[t], rowmax[BM + t]);
        __hip_atomic_fetch_max(rq.amax + row_t, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // the atomics have completed (vmcnt(0)) before any lane of the block goes on
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));
    __syncthreads();
    if (t == 0) {
        // 3. wait for the stripe's other tiles (the last to arrive need not)
        const uint32_t before = __hip_atomic_fetch_add(rq.arrived + tm, 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        while (before + 1 < (uint32_t)tiles_n &&
               __hip_atomic_load(rq.arrived + tm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
                   (uint32_t)tiles_n) {
            __builtin_amdgcn_s_sleep(2);
            if (__builtin_amdgcn_s_memrealtime() - t0 > kRqWaitTicks) {
                __hip_atomic_fetch_add(&g_rq_timeouts, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // the rows' inverse scales replace the row scales in LDS (last read in step 1);
    // the clamp is needed only if a row max lies outside [2^-14, 65504]
    bool wide;
    {
        const uint32_t bits = __hip_atomic_load(rq.amax + min(row_t, M - 1), __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        const float amax = fmaxf(__uint_as_float(bits), 1e-8f);
        esa[t] = 127.f / amax;
        if (tn == 0 && row_t < M) rq.scales[row_t] = amax / 127.f;
        wide = __syncthreads_or(!(amax >= 0x1p-14f && amax <= 65504.f)) != 0;
    }
    // 4. codes
    if (wide) rq_store_codes<true>(lds, esa, rq, M, N, m0, n0);
    else rq_store_codes<false>(lds, esa, rq, M, N, m0, n0);
}

// BKN: Bt is B stored [K][N] (row stride N), read without a transpose.
template <int EPI, bool BKN = false>
__global__ __launch_bounds__(kThreads, 1) void gemm_i8_rq_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ Bt, int M, int N, int K,
    int tiles_m, int tiles_n, EpiParams p, RqParams rq) {
    static_assert(EPI == EPI_GELU_F16 || EPI == EPI_F16, "requantizing epilogues only");
    extern __shared__ __align__(16) char lds[];
    int tm, tn;
    rq_tile_coords(blockIdx.x, tiles_m, tiles_n, rq, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x;
    const float pre_sa = p.sa[(size_t)min(m0 + t, M - 1) * p.sa_stride];
    const float pre_sb = p.sb[(size_t)min(n0 + t, N - 1) * p.sb_stride];
    const float pre_b = p.bias != nullptr ? p.bias[min(n0 + t, N - 1)] : 0.f;
    v16i acc[TM][TN];
    const int ldb = BKN ? N : K;
    if (m0 + BM <= M && n0 + BN <= N && K % BK == 0)
        mainloop<false, true, BKN>(acc, A, Bt, M, N, K, K, ldb, m0, n0, lds);
    else
        mainloop<true, true, BKN>(acc, A, Bt, M, N, K, K, ldb, m0, n0, lds);
    epilogue_rq<EPI>(acc, rq, M, N, m0, n0, tm, tn, tiles_n, pre_sa, pre_sb, pre_b, lds);
}

// Zeroes n dwords (the fused requant's amax and arrival counters) before the GEMMs.
__global__ __launch_bounds__(256) void rq_clear_kernel(uint32_t* __restrict__ p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

// ------------------------------------------------------------ mid-size grids
// gemm_i8_mid_kernel<EPI>: 128 x 128 output tiles for GEMMs whose 256 x 256
// grid leaves CUs idle (T = 4096 at d_model 1024: GEMM2 has 16 x 4 big tiles
// for 256 CUs).  Four waves in a 2 x 2 grid each own 64 x 64 (2 x 2 MFMA
// tiles of 32 x 32 x 32); A and Bt go global -> VGPR -> LDS in the big
// kernel's padded layout, double-buffered, the next K-step's loads in flight
// during the current one.  75 KiB of LDS: two blocks per CU, whose waves hide
// each other's waits.  Half the MFMA work per fragment read of the big tile,
// so it runs only where the big grid is too small.  Same epilogue code and
// bytes as gemm_i8_kernel, with one absmax partial per row and 128 columns.
constexpr int kMidB = 128, kMidW = 64, kMidT = kMidW / 32;
constexpr int kMidAStage = kMidB * LDS_STRIDE;
constexpr int kMidStage = 2 * kMidAStage;
constexpr int kMidLds = 2 * kMidStage;
constexpr int kMidEpiLds = kMidLds + 3 * kMidB * 4;
constexpr int kMidChunks = kMidB * kChunksPerRow / kThreads;
static_assert(kMidChunks == 4 && 2 * kMidEpiLds <= 160 * 1024, "two blocks per CU");

template <bool EDGE>
__device__ __forceinline__ void mid_mainloop(v16i (&acc)[kMidT][kMidT],
                                             const int8_t* __restrict__ A,
                                             const int8_t* __restrict__ Bt, int M, int N, int K,
                                             int m0, int n0, char* lds) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
    for (int i = 0; i < kMidT; ++i)
#pragma unroll
        for (int j = 0; j < kMidT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    const int nk = (K + BK - 1) / BK;
    const int a_off = (wm * kMidW + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 16;
    const int b_off = kMidAStage + (wn * kMidW + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 16;
    int4 fa[kMidChunks], fb[kMidChunks];
    // chunk c = t + 256 i of a 128 x 128-byte operand tile: row c / 8, bytes (c % 8) * 16;
    // rows past the matrix and K past the end load clamped addresses, zeroed on EDGE
    auto load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kMidChunks; ++i) {
            const int c = threadIdx.x + i * kThreads;
            const int row = c / kChunksPerRow, kc = (c % kChunksPerRow) * 16;
            const int gk = min(k0 + kc, K - 16);
            fa[i] = *reinterpret_cast<const int4*>(A + (size_t)min(m0 + row, M - 1) * K + gk);
            fb[i] = *reinterpret_cast<const int4*>(Bt + (size_t)min(n0 + row, N - 1) * K + gk);
        }
    };
    auto store = [&](char* stage, int k0) {
#pragma unroll
        for (int i = 0; i < kMidChunks; ++i) {
            const int c = threadIdx.x + i * kThreads;
            const int row = c / kChunksPerRow, kc = (c % kChunksPerRow) * 16;
            int4 va = fa[i], vb = fb[i];
            if constexpr (EDGE) {
                const bool kok = k0 + kc < K;
                if (!(kok && m0 + row < M)) va = make_int4(0, 0, 0, 0);
                if (!(kok && n0 + row < N)) vb = make_int4(0, 0, 0, 0);
            }
            *reinterpret_cast<int4*>(stage + row * LDS_STRIDE + kc) = va;
            *reinterpret_cast<int4*>(stage + kMidAStage + row * LDS_STRIDE + kc) = vb;
        }
    };
    // fragments of k-slice s of a stage: rows (l % 32) of the wave's two 32-row
    // blocks of A and of Bt, 16-byte half (l / 32)
    auto read = [&](v4i (&a)[kMidT], v4i (&b)[kMidT], const char* stage, int s) {
#pragma unroll
        for (int i = 0; i < kMidT; ++i)
            a[i] = *reinterpret_cast<const v4i*>(stage + a_off + i * 32 * LDS_STRIDE + s * 32);
#pragma unroll
        for (int j = 0; j < kMidT; ++j)
            b[j] = *reinterpret_cast<const v4i*>(stage + b_off + j * 32 * LDS_STRIDE + s * 32);
    };
    auto mma = [&](const v4i (&a)[kMidT], const v4i (&b)[kMidT]) {
#pragma unroll
        for (int i = 0; i < kMidT; ++i)
#pragma unroll
            for (int j = 0; j < kMidT; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    };
    load(0);
    store(lds, 0);
    if (nk > 1) load(BK);
    __syncthreads();
    v4i a[2][kMidT], b[2][kMidT];
    read(a[0], b[0], lds, 0);
    // Step kt reads buffer kt & 1 and writes buffer (kt + 1) & 1, whose last
    // reads (step kt - 1) finished before that step's barrier.  The fragments
    // of slice 3 are in registers before the barrier, so its MFMAs run after
    // it, while the reads of the next stage's slice 0 are in flight.
    for (int kt = 0; kt < nk; ++kt) {
        const char* cur = lds + (kt & 1) * kMidStage;
        char* nxt = lds + ((kt + 1) & 1) * kMidStage;
        read(a[1], b[1], cur, 1);
        mma(a[0], b[0]);
        read(a[0], b[0], cur, 2);
        mma(a[1], b[1]);
        read(a[1], b[1], cur, 3);
        mma(a[0], b[0]);
        if (kt + 1 < nk) store(nxt, (kt + 1) * BK);
        if (kt + 2 < nk) load((kt + 2) * BK);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 1 < nk) read(a[0], b[0], nxt, 0);
        mma(a[1], b[1]);
    }
}

template <int EPI>
__global__ __launch_bounds__(kThreads, 2) void gemm_i8_mid_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ Bt, int M, int N, int K,
    int tiles_m, int tiles_n, EpiParams p) {
    static_assert(EPI != EPI_I32, "fused epilogues only");
    extern __shared__ __align__(16) char lds[];
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * kMidB, n0 = tn * kMidB;
    // threads t and t + 128 load row / column t's scales (clamped, unconditional);
    // the epilogue keeps those of t < 128
    const int t = threadIdx.x & (kMidB - 1);
    const float pre_sa = p.sa[(size_t)min(m0 + t, M - 1) * p.sa_stride];
    const float pre_sb = p.sb[(size_t)min(n0 + t, N - 1) * p.sb_stride];
    const float pre_b = p.bias != nullptr ? p.bias[min(n0 + t, N - 1)] : 0.f;
    v16i acc[kMidT][kMidT];
    if (m0 + kMidB <= M && n0 + kMidB <= N && K % BK == 0)
        mid_mainloop<false>(acc, A, Bt, M, N, K, m0, n0, lds);
    else
        mid_mainloop<true>(acc, A, Bt, M, N, K, m0, n0, lds);
    epilogue_tile<EPI, kMidT, kMidT, kMidW, kMidW, kMidB, kMidLds>(acc, p, M, N, m0, n0, tn,
                                                                   pre_sa, pre_sb, pre_b, lds);
}

// The MLP's GEMM2 over the fp16 hidden A16 [M][K] itself, with no
// requantization pass and no int8 hidden in memory: each block reduces its 256
// rows' absmax from GEMM1's partials (pmax1, tn1 per row) as
// requant_rows_kernel does, quantizes A on its way to LDS (mainloop_a16) and
// runs gemm_i8_kernel<EPI_F16>'s epilogue with the hidden row scale
// amax / 127.
constexpr int kA16LdsBytes = kEpiLdsBytes + BM * 4;  // + the rows' 127 / amax

__global__ __launch_bounds__(kThreads, 1) void gemm_i8_a16_kernel(
    const uint16_t* __restrict__ A16, const int8_t* __restrict__ Bt, int M, int N, int K,
    int tiles_m, int tiles_n, const float* __restrict__ pmax1, int tn1, EpiParams p) {
    extern __shared__ __align__(16) char lds[];
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int t = threadIdx.x;
    const int row = min(m0 + t, M - 1);
    float mx = 0.f;
    for (int j = 0; j < tn1; ++j) mx = fmaxf(mx, pmax1[(size_t)j * M + row]);
    const float amax = fmaxf(mx, 1e-8f);
    const float pre_sa = amax / 127.f;
    const float pre_sb = p.sb[(size_t)min(n0 + t, N - 1) * p.sb_stride];
    float* einv = reinterpret_cast<float*>(lds + kEpiLdsBytes);
    einv[t] = 127.f / amax;
    // a row max past the fp16 range: some h may be infinite, so clamp before rounding
    const bool exact = __syncthreads_or(!(amax <= 65504.f)) != 0;
    float inv[kChunks];
#pragma unroll
    for (int i = 0; i < kChunks; ++i) inv[i] = einv[(t + i * kThreads) / kChunksPerRow];
    v16i acc[TM][TN];
    const bool interior = m0 + BM <= M && n0 + BN <= N && K % BK == 0;
    if (exact) {
        if (interior) mainloop_a16<false, true>(acc, A16, Bt, M, N, K, K, K, m0, n0, lds, inv);
        else mainloop_a16<true, true>(acc, A16, Bt, M, N, K, K, K, m0, n0, lds, inv);
    } else {
        if (interior) mainloop_a16<false, false>(acc, A16, Bt, M, N, K, K, K, m0, n0, lds, inv);
        else mainloop_a16<true, false>(acc, A16, Bt, M, N, K, K, K, m0, n0, lds, inv);
    }
    epilogue_tile<EPI_F16>(acc, p, M, N, m0, n0, tn, pre_sa, pre_sb, 0.f, lds);
}

// ---------------------------------------------------------------- split-K path

constexpr int kSkN = 128;       // output columns per block (4 waves x 32)
constexpr int kSkM = 128;       // output rows per block (4 MFMA row tiles)
constexpr int kSkK = 128;       // K bytes per step
constexpr int kSkStride = kSkK + 16;  // padded LDS row of the A tile
constexpr int kSkLds = 2 * kSkM * kSkStride;

// P[split][M][N] (int32) = A[m0:m0+128, k range] . Bt[n0:n0+128, k range]^T.
// grid = (N tiles, splits, M tiles); each wave owns 32 columns and all 128 rows
// (4 x 32x32x32 MFMA tiles).  The A tile goes through LDS (shared by the four
// waves); B fragments are loaded straight from global memory (each column is
// used by one wave only).  K is a multiple of 32; rows >= M read as zero.
__global__ __launch_bounds__(256) void gemm_i8_splitk_kernel(
    const int8_t* __restrict__ A, const int8_t* __restrict__ Bt, int32_t* __restrict__ P,
    int M, int N, int K, int k_per_split) {
    extern __shared__ __align__(16) char lds[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * kSkN, m0 = blockIdx.z * kSkM;
    const int kb = blockIdx.y * k_per_split;
    const int ke = min(K, kb + k_per_split);
    const int ncol = n0 + wave * 32 + (lane & 31);
    const int8_t* brow = Bt + (size_t)min(ncol, N - 1) * K;
    v16i acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0;

    // A staging: 128 rows x 128 bytes = 1024 chunks of 16 B, 4 per thread
    int4 ar[4];
    auto load_a = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = threadIdx.x + i * 256;
            const int row = c >> 3, kc = (c & 7) * 16;
            const int gk = min(k0 + kc, K - 16);
            ar[i] = *reinterpret_cast<const int4*>(A + (size_t)min(m0 + row, M - 1) * K + gk);
        }
    };
    auto store_a = [&](char* buf, int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = threadIdx.x + i * 256;
            const int row = c >> 3, kc = (c & 7) * 16;
            int4 v = ar[i];
            if (!(m0 + row < M && k0 + kc < ke)) v = make_int4(0, 0, 0, 0);
            *reinterpret_cast<int4*>(buf + row * kSkStride + kc) = v;
        }
    };
    const int nsteps = (ke - kb + kSkK - 1) / kSkK;
    load_a(kb);
    for (int st = 0; st < nsteps; ++st) {
        const int k0 = kb + st * kSkK;
        char* buf = lds + (st & 1) * (kSkM * kSkStride);
        store_a(buf, k0);
        // B fragments of this step: column ncol, bytes k0 + 32 s + 16 (lane / 32)
        v4i bf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kk = k0 + 32 * s + 16 * (lane >> 5);
            bf[s] = kk < ke ? *reinterpret_cast<const v4i*>(brow + kk) : v4i{0, 0, 0, 0};
        }
        if (st + 1 < nsteps) load_a(k0 + kSkK);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if (k0 + 32 * s >= ke) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const v4i af = *reinterpret_cast<const v4i*>(
                    buf + (32 * i + (lane & 31)) * kSkStride + 32 * s + 16 * (lane >> 5));
                acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[s], acc[i], 0, 0, 0);
            }
        }
    }
    if (ncol >= N) return;
    int32_t* Pp = P + (size_t)blockIdx.y * M * N;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + 32 * i + acc_row(r, lane);
            if (row < M) Pp[(size_t)row * N + ncol] = acc[i][r];
        }
}

// acc = sum of the split partials (exact int32), then gemm_i8_kernel's
// epilogue math for EPI (same expressions) and the fp16 store.  Block (x, y)
// covers columns [256 x, 256 x + 256) of row y and writes that chunk's absmax
// to pmax[x][row], like one 256-column tile of gemm_i8_kernel.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_epilogue_kernel(const int32_t* __restrict__ P,
                                                              int splits, int M, int N,
                                                              EpiParams p) {
    __shared__ float red[4];
    const int row = blockIdx.y;
    const int n = blockIdx.x * 256 + threadIdx.x;
    float m = 0.f;
    if (n < N) {
        const int32_t* col = P + (size_t)row * N + n;
        const size_t plane = (size_t)M * N;
        int acc = 0;
#pragma unroll 8
        for (int sp = 0; sp < splits; ++sp) acc += col[sp * plane];
        float v = static_cast<float>(acc) * p.sa[(size_t)row * p.sa_stride] *
                  p.sb[(size_t)n * p.sb_stride];
        if constexpr (EPI == EPI_GELU_F16)
            v = gelu_tanh(v + (p.bias != nullptr ? p.bias[n] : 0.f));
        m = fabsf(v);
        p.c16[(size_t)row * p.ldc + n] = f32_to_f16_bits(v);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0)
        p.pmax[(size_t)blockIdx.x * M + row] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// ---------------------------------------------------------------- few tokens
// Skinny GEMM for small GEMMs (decode-time MLPs): a block owns one 32 x 32
// output tile (grid = N/32 column blocks x M/32 row blocks) over the whole K,
// and its four waves take a quarter of K each.  MFMA operands come straight
// from global memory: the tile's 32 rows of A and 32 rows of Bt, 16 bytes per
// lane, two groups of four 32-deep k slices in flight.  The four int32
// partial tiles meet in LDS and the block's 256 threads apply the epilogue,
// writing one absmax partial per (32-column block, row).  No partial sums
// leave the chip; split-K over blocks (above) would write them to memory.
// Rows past M read row M-1 and are not stored.
//
//
// It runs at ~3 us + 7 us per 2^30 multiply-adds on MI355X (latency-bound
// loads; the tiles re-read A and Bt through L2, ~MNK/16 bytes).  Per GEMM,
// measured against split-K and the 256 x 256 kernel at d_model 512..4096 and
// T 1..2048, it wins up to M N K = 2^31, and up to 2^32 above 512 rows (no
// split-K there) when the 256 x 256 grid would have fewer than 64 tiles.
constexpr int kSkinnyN = 32;
constexpr int kSkinnyLds = 4 * 32 * kSkinnyN * 4 + 32 * 4;  // partials, row scales

inline bool use_skinny(int M, int N, int K) {
    if (N % kSkinnyN != 0 || K % 512 != 0) return false;
    const long long mnk = (long long)M * N * K;
    const long long big_tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    return mnk <= (1LL << 31) || (M > 4 * kSkM && big_tiles < 64 && mnk <= (1LL << 32));
}


__device__ __forceinline__ void skinny_load(v4i (&b)[4], v4i (&a)[4], const int8_t* arow,
                                            const int8_t* brow, int k) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        b[u] = *reinterpret_cast<const v4i*>(brow + k + 32 * u);
        a[u] = *reinterpret_cast<const v4i*>(arow + k + 32 * u);
    }
}

__device__ __forceinline__ void skinny_mfma(v16i& acc, const v4i (&b)[4], const v4i (&a)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u], b[u], acc, 0, 0, 0);
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_i8_skinny_kernel(const int8_t* __restrict__ A,
                                                             const int8_t* __restrict__ Bt,
                                                             int M, int N, int K, EpiParams p) {
    extern __shared__ __align__(16) char lds[];
    (void)N;  // the grid covers the columns exactly: N % kSkinnyN == 0 (use_skinny)
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * kSkinnyN;
    const int m0 = blockIdx.y * 32;
    const int c = threadIdx.x & 31;
    const int col = n0 + c;
    // epilogue operands first, so the K loop hides their latency
    const float pre_sa = p.sa[(size_t)min(m0 + c, M - 1) * p.sa_stride];
    const float sb = p.sb[(size_t)col * p.sb_stride];
    const float bias = p.bias != nullptr ? p.bias[col] : 0.f;

    const int kq = K / 4;  // this wave's quarter of K, a multiple of 128
    const int koff = wave * kq + (lane >> 5) * 16;
    const int8_t* arow = A + (size_t)min(m0 + (lane & 31), M - 1) * K + koff;
    const int8_t* brow = Bt + (size_t)(n0 + (lane & 31)) * K + koff;
    v16i acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0;
    // two groups of four k slices in flight: group g+1 loads while g runs
    v4i b0[4], a0[4], b1[4], a1[4];
    skinny_load(b0, a0, arow, brow, 0);
    for (int k = 0; k < kq; k += 256) {
        if (k + 128 < kq) skinny_load(b1, a1, arow, brow, k + 128);
        skinny_mfma(acc, b0, a0);
        if (k + 128 >= kq) break;
        if (k + 256 < kq) skinny_load(b0, a0, arow, brow, k + 256);
        skinny_mfma(acc, b1, a1);
    }
    // partials part[wave][row][col] (row acc_row(r), column lane % 32), row scales
    int* part = reinterpret_cast<int*>(lds);
    float* esa = reinterpret_cast<float*>(lds + 4 * 32 * kSkinnyN * 4);
#pragma unroll
    for (int r = 0; r < 16; ++r) part[(wave * 32 + acc_row(r, lane)) * kSkinnyN + (lane & 31)] = acc[r];
    if (threadIdx.x < 32) esa[threadIdx.x] = pre_sa;
    __syncthreads();
    // epilogue: thread t takes column t % 32 of rows t / 32 + 8 j (j < 4); the
    // 32 lanes of a half-wave share a row: its absmax by DPP inside each 16-lane
    // row and v_permlane16_swap across the two (VALU only)
    float v[4];
    int mx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int rl = (threadIdx.x >> 5) + 8 * j;
        const int s = part[rl * kSkinnyN + c] + part[(32 + rl) * kSkinnyN + c] +
                      part[(64 + rl) * kSkinnyN + c] + part[(96 + rl) * kSkinnyN + c];
        v[j] = epi_value<EPI>(s, esa[rl], sb, bias);
        mx[j] = __float_as_int(fabsf(v[j]));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = max(mx[j], dpp_xor1(mx[j]));
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = max(mx[j], dpp_xor2(mx[j]));
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = max(mx[j], dpp_half_mirror(mx[j]));
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = max(mx[j], dpp_row_mirror(mx[j]));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const auto sw = __builtin_amdgcn_permlane16_swap(mx[j], mx[j], false, false);
        mx[j] = max((int)sw[0], (int)sw[1]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = m0 + (threadIdx.x >> 5) + 8 * j;
        if (row < M) {
            p.c16[(size_t)row * p.ldc + col] = f32_to_f16_bits(v[j]);
            if (c == 0) p.pmax[(size_t)blockIdx.x * M + row] = __int_as_float(mx[j]);
        }
    }
}

template <int EPI>
int launch_gemm_skinny(const int8_t* A, const int8_t* Bt, int M, int N, int K, const EpiParams& p,
                       hipStream_t stream) {
    const dim3 grid(N / kSkinnyN, (M + 31) / 32);
    gemm_i8_skinny_kernel<EPI><<<grid, 256, kSkinnyLds, stream>>>(A, Bt, M, N, K, p);
    return check_launch("gemm_i8_skinny_kernel");
}

// Split plan for an M x N x K GEMM: run split-K when the 256 x 256 grid would
// have fewer tiles than the device has CUs (256 on MI355X).
struct SplitKPlan {
    bool use;
    int splits, k_per_split, tiles_n, tiles_m;
};

inline SplitKPlan splitk_plan(int M, int N, int K) {
    SplitKPlan pl{};
    const long long big_tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (big_tiles >= 256 || K % 32 != 0 || M > 4 * kSkM) return pl;
    pl.tiles_n = (N + kSkN - 1) / kSkN;
    pl.tiles_m = (M + kSkM - 1) / kSkM;
    const int ksteps = (K + kSkK - 1) / kSkK;
    const int want = (int)std::max<long long>(1, (512 + pl.tiles_n * pl.tiles_m - 1) /
                                                     (pl.tiles_n * pl.tiles_m));
    const int steps_per = (ksteps + std::min(want, ksteps) - 1) / std::min(want, ksteps);
    pl.k_per_split = steps_per * kSkK;
    pl.splits = (K + pl.k_per_split - 1) / pl.k_per_split;
    pl.use = true;
    return pl;
}

// The 128 x 128 kernel takes the GEMMs that the few-token paths leave and whose
// 256 x 256 grid has at most 128 tiles: then its 4x as many tiles fit one round
// of two blocks on each of the 256 CUs.  Measured per MLP (d_model 1024, d_ff
// 4096, prepacked): T = 2048 86 -> 57 us, T = 4096 99 -> 82 us, T = 8192 (128
// big tiles in GEMM2) 145 -> 140 us; at 192 big tiles (T = 12288) it lost 11%.
constexpr int kMidMaxBigTiles = 128;

inline bool use_mid(int M, int N, int K) {
    if (use_skinny(M, N, K) || splitk_plan(M, N, K).use) return false;
    const long long big_tiles = (long long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    return big_tiles <= kMidMaxBigTiles;
}

// Absmax partials per row that the GEMM's epilogue leaves (requant reads them).
inline int epi_tiles(int M, int N, int K) {
    if (use_skinny(M, N, K)) return N / kSkinnyN;
    return use_mid(M, N, K) ? (N + kMidB - 1) / kMidB : (N + BN - 1) / BN;
}

inline size_t splitk_partial_bytes(int M, int N, int K) {
    const SplitKPlan pl = splitk_plan(M, N, K);
    return pl.use ? (size_t)pl.splits * M * N * 4 : 0;
}

template <int EPI>
int launch_gemm_splitk(const int8_t* A, const int8_t* Bt, int M, int N, int K,
                       const SplitKPlan& pl, int32_t* partial, const EpiParams& p,
                       hipStream_t stream) {
    const dim3 grid(pl.tiles_n, pl.splits, pl.tiles_m);
    gemm_i8_splitk_kernel<<<grid, 256, kSkLds, stream>>>(A, Bt, partial, M, N, K,
                                                         pl.k_per_split);
    int st = check_launch("gemm_i8_splitk_kernel");
    if (st != INT8K_OK) return st;
    splitk_epilogue_kernel<EPI><<<dim3((N + 255) / 256, M), 256, 0, stream>>>(partial, pl.splits,
                                                                              M, N, p);
    return check_launch("splitk_epilogue_kernel");
}

// One block per row: reduce the row's absmax partials, then requantize the
// fp16 row to int8 with scale max(amax,1e-8)/127 (quantize_rows semantics).
// With `tensor_amax` set, that single value is used for every row instead
// and `scales` receives it once (per-tensor output quantization).
__global__ __launch_bounds__(256) void requant_rows_kernel(
    const uint16_t* __restrict__ h, int ldh, const float* __restrict__ pmax, int tiles_n,
    const float* __restrict__ tensor_amax, int8_t* __restrict__ q, int ldq,
    float* __restrict__ scales, int M, int N) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    float amax;
    if (tensor_amax != nullptr) {
        amax = *tensor_amax;
    } else {
        float m = 0.f;
        for (int t = threadIdx.x; t < tiles_n; t += 256) m = fmaxf(m, pmax[(size_t)t * M + row]);
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        __syncthreads();
        amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    }
    amax = fmaxf(amax, 1e-8f);
    const float inv = 127.f / amax;
    if (threadIdx.x == 0 && (tensor_amax == nullptr || row == 0))
        scales[tensor_amax == nullptr ? row : 0] = amax / 127.f;
    const uint16_t* hr = h + (size_t)row * ldh;
    int8_t* qr = q + (size_t)row * ldq;
    auto quant = [inv](uint16_t bits) -> int {
        const float f = __half2float(__ushort_as_half(bits)) * inv;
        return static_cast<int>(__builtin_rintf(fminf(fmaxf(f, -128.f), 127.f)));
    };
    if ((N & 7) == 0 && (ldh & 7) == 0 && (ldq & 7) == 0) {
        // the fp16 rows are read once, here (non-temporal), and several loads per
        // thread go out before the first one is used
        typedef uint32_t v4u __attribute__((ext_vector_type(4)));
#pragma unroll 4
        for (int c = threadIdx.x * 8; c < N; c += 256 * 8) {
            const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(hr + c));
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t lo = 0, hi = 0;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                lo |= (uint32_t)(quant(w[e] & 0xffff) & 0xff) << (16 * e);
                lo |= (uint32_t)(quant(w[e] >> 16) & 0xff) << (16 * e + 8);
                hi |= (uint32_t)(quant(w[2 + e] & 0xffff) & 0xff) << (16 * e);
                hi |= (uint32_t)(quant(w[2 + e] >> 16) & 0xff) << (16 * e + 8);
            }
            *reinterpret_cast<uint2*>(qr + c) = make_uint2(lo, hi);
        }
    } else {
        for (int c = threadIdx.x; c < N; c += 256) qr[c] = (int8_t)quant(hr[c]);
    }
}

// requant_rows_kernel for rows of up to 2048 columns (N % 8 == 0, 16-byte
// aligned rows): one wave per row, four rows per block, so short rows keep
// every lane busy and the reductions stay inside the wave.
__global__ __launch_bounds__(256) void requant_rows_wave_kernel(
    const uint16_t* __restrict__ h, int ldh, const float* __restrict__ pmax, int tiles_n,
    const float* __restrict__ tensor_amax, int8_t* __restrict__ q, int ldq,
    float* __restrict__ scales, int M, int N) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    float amax;
    if (tensor_amax != nullptr) {
        amax = *tensor_amax;
    } else {
        float m = 0.f;
        for (int t = lane; t < tiles_n; t += 64) m = fmaxf(m, pmax[(size_t)t * M + row]);
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
        amax = m;
    }
    amax = fmaxf(amax, 1e-8f);
    const float inv = 127.f / amax;
    if (lane == 0 && (tensor_amax == nullptr || row == 0))
        scales[tensor_amax == nullptr ? row : 0] = amax / 127.f;
    const uint16_t* hr = h + (size_t)row * ldh;
    int8_t* qr = q + (size_t)row * ldq;
    auto quant = [inv](uint16_t bits) -> int {
        const float f = __half2float(__ushort_as_half(bits)) * inv;
        return static_cast<int>(__builtin_rintf(fminf(fmaxf(f, -128.f), 127.f)));
    };
    for (int c = lane * 8; c < N; c += 64 * 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(hr + c);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            lo |= (uint32_t)(quant(w[e] & 0xffff) & 0xff) << (16 * e);
            lo |= (uint32_t)(quant(w[e] >> 16) & 0xff) << (16 * e + 8);
            hi |= (uint32_t)(quant(w[2 + e] & 0xffff) & 0xff) << (16 * e);
            hi |= (uint32_t)(quant(w[2 + e] >> 16) & 0xff) << (16 * e + 8);
        }
        *reinterpret_cast<uint2*>(qr + c) = make_uint2(lo, hi);
    }
}

// Launches the requant pass for M rows of N columns: one wave per row for rows
// of up to 2048 columns when there are enough rows to fill the chip (at
// T = 16384, 1024 columns: 17.1 -> 12.3 us), else one block per row.
int launch_requant(const uint16_t* h, int ldh, const float* pmax, int tiles_n,
                   const float* tensor_amax, int8_t* q, int ldq, float* scales, int M, int N,
                   hipStream_t s) {
    if (M >= 512 && N <= 2048 && N % 8 == 0 && ldh % 8 == 0 && ldq % 8 == 0 &&
        aligned_to(h, 16) && aligned_to(q, 8)) {
        requant_rows_wave_kernel<<<(M + 3) / 4, 256, 0, s>>>(h, ldh, pmax, tiles_n, tensor_amax,
                                                             q, ldq, scales, M, N);
        return check_launch("requant_rows_wave_kernel");
    }
    requant_rows_kernel<<<M, 256, 0, s>>>(h, ldh, pmax, tiles_n, tensor_amax, q, ldq, scales, M,
                                          N);
    return check_launch("requant_rows_kernel");
}

// Max over all partials (per-tensor output scale), one block.
__global__ __launch_bounds__(256) void tensor_absmax_kernel(const float* __restrict__ pmax,
                                                            size_t n, float* __restrict__ out) {
    __shared__ float red[4];
    float m = 0.f;
    for (size_t i = threadIdx.x; i < n; i += 256) m = fmaxf(m, pmax[i]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) *out = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// dst[C][R] = src[R][C]^T in 128 x 128-byte tiles.  Interior tiles of 16-byte
// aligned matrices (vec): each thread loads 16 bytes of 4 source rows (8 threads
// cover a row's 128 bytes), the tile goes to LDS as dwords (row stride 33
// dwords), each thread reads the 4-column dwords of 16 source rows, transposes
// them in 4 x 4 byte blocks with v_perm, and stores 16 bytes of 4 destination
// rows (8 threads cover a row's 128 bytes).  Other tiles go byte by byte.
constexpr int kTrTile = 128;
constexpr int kTrStride = kTrTile / 4 + 1;  // LDS dwords per source row

__global__ __launch_bounds__(256) void transpose_i8_kernel(const int8_t* __restrict__ src,
                                                           int8_t* __restrict__ dst, int R, int C,
                                                           int vec_ok) {
    __shared__ uint32_t tile[kTrTile * kTrStride];
    const int r0 = blockIdx.y * kTrTile, c0 = blockIdx.x * kTrTile;
    const int t = threadIdx.x;
    if (vec_ok && r0 + kTrTile <= R && c0 + kTrTile <= C) {
        const int cw = (t & 7) * 4;  // first dword of this thread's 16 bytes
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = (t >> 3) + 32 * i;
            const uint4 v = *reinterpret_cast<const uint4*>(src + (size_t)(r0 + r) * C + c0 + 4 * cw);
            uint32_t* row = tile + r * kTrStride + cw;
            row[0] = v.x;
            row[1] = v.y;
            row[2] = v.z;
            row[3] = v.w;
        }
        __syncthreads();
        // destination rows 4a .. 4a+3 (source columns), bytes = source rows 16b .. 16b+15
        const int a = t >> 3, b = t & 7;
        uint32_t w[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = tile[(16 * b + i) * kTrStride + a];
        uint32_t o[4][4];  // [destination row j][dword g: source rows 16b + 4g .. +3]
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            // {w0.bk, w1.bk, w0.bk', w1.bk'} pairs, then the 4-byte column of byte j
            const uint32_t lo01 = __builtin_amdgcn_perm(w[4 * g + 1], w[4 * g], 0x05010400u);
            const uint32_t hi01 = __builtin_amdgcn_perm(w[4 * g + 1], w[4 * g], 0x07030602u);
            const uint32_t lo23 = __builtin_amdgcn_perm(w[4 * g + 3], w[4 * g + 2], 0x05010400u);
            const uint32_t hi23 = __builtin_amdgcn_perm(w[4 * g + 3], w[4 * g + 2], 0x07030602u);
            o[0][g] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
            o[1][g] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
            o[2][g] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
            o[3][g] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<uint4*>(dst + (size_t)(c0 + 4 * a + j) * R + r0 + 16 * b) =
                make_uint4(o[j][0], o[j][1], o[j][2], o[j][3]);
        return;
    }
    int8_t* tb = reinterpret_cast<int8_t*>(tile);
    constexpr int kB = kTrStride * 4;  // bytes per LDS row
    for (int i = t; i < kTrTile * kTrTile; i += 256) {
        const int r = i / kTrTile, c = i % kTrTile;
        if (r0 + r < R && c0 + c < C) tb[r * kB + c] = src[(size_t)(r0 + r) * C + c0 + c];
    }
    __syncthreads();
    for (int i = t; i < kTrTile * kTrTile; i += 256) {
        const int c = i / kTrTile, r = i % kTrTile;
        if (r0 + r < R && c0 + c < C) dst[(size_t)(c0 + c) * R + r0 + r] = tb[r * kB + c];
    }
}

// The 256 x 256 kernels address each operand through a buffer resource with
// 32-bit offsets: operands of 4 GiB or more are not taken.
inline int check_tiled_operands(int M, int N, int K) {
    if ((size_t)M * K >= (1ull << 32) || (size_t)N * K >= (1ull << 32)) {
        set_last_error_text("int8 GEMM operand of 4 GiB or more");
        return INT8K_ERR_UNSUPPORTED;
    }
    return INT8K_OK;
}

template <int EPI, bool BKN = false>
int launch_gemm(const int8_t* A, const int8_t* Bt, int M, int N, int K, const EpiParams& p,
                hipStream_t stream) {
    if (int st = check_tiled_operands(M, N, K)) return st;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    gemm_i8_kernel<EPI, BKN>
        <<<tiles_m * tiles_n, kThreads, EPI == EPI_I32 ? LDS_BYTES : kEpiLdsBytes, stream>>>(
            A, Bt, M, N, K, K, BKN ? N : K, tiles_m, tiles_n, p);
    return check_launch("gemm_i8_kernel");
}

template <int EPI>
int launch_gemm_mid(const int8_t* A, const int8_t* Bt, int M, int N, int K, const EpiParams& p,
                    hipStream_t stream) {
    const int tiles_m = (M + kMidB - 1) / kMidB, tiles_n = (N + kMidB - 1) / kMidB;
    gemm_i8_mid_kernel<EPI><<<tiles_m * tiles_n, kThreads, kMidEpiLds, stream>>>(
        A, Bt, M, N, K, tiles_m, tiles_n, p);
    return check_launch("gemm_i8_mid_kernel");
}

// Tile order of a fused-requant GEMM: per group of stripes, each XCD takes a panel
// of pm stripes x pn column tiles (about 32 tiles, one round of its CUs) with
// the smallest pm + pn, which is the operand bytes its L2 holds per K-step.  A
// stripe's pn tiles on one XCD must be resident together, so pn stays at most
// kRqMaxPanelCols (half an XCD's 32 CUs); shapes with no such panel take the
// stripe-major order, which spreads a stripe over the XCDs round-robin.
constexpr int kRqMaxPanelCols = 16;

RqParams rq_layout(int tiles_m, int tiles_n) {
    RqParams r{};
    r.gs = 1;
    r.xm = 1;
    r.xn = 0;
    int best = 1 << 30;
    for (int xn = 8; xn >= 1; xn >>= 1) {
        if (tiles_n % xn != 0) continue;
        const int pn = tiles_n / xn, xm = kNumXcd / xn;
        const int pm = std::max(1, 32 / pn);
        if (pn <= kRqMaxPanelCols && pm + pn < best && pm * xm <= std::max(tiles_m, xm)) {
            best = pm + pn;
            r.xn = xn;
            r.xm = xm;
            r.gs = pm * xm;
        }
    }
    return r;
}

// A GEMM with the per-token requantization in its epilogue: codes q [M][N] and
// row scales; amax [M] and arrived [tiles_m] must be zero.
template <int EPI, bool BKN = false>
int launch_gemm_rq(const int8_t* A, const int8_t* Bt, int M, int N, int K, const EpiParams& p,
                   int8_t* q, float* scales, uint32_t* amax, uint32_t* arrived,
                   hipStream_t stream) {
    if (int st = check_tiled_operands(M, N, K)) return st;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    RqParams rq = rq_layout(tiles_m, tiles_n);
    rq.q = q;
    rq.ldq = N;
    rq.scales = scales;
    rq.amax = amax;
    rq.arrived = arrived;
    gemm_i8_rq_kernel<EPI, BKN><<<tiles_m * tiles_n, kThreads, kEpiLdsBytes, stream>>>(
        A, Bt, M, N, K, tiles_m, tiles_n, p, rq);
    return check_launch("gemm_i8_rq_kernel");
}

int launch_transpose(const int8_t* src, int8_t* dst, int R, int C, hipStream_t stream) {
    const dim3 grid((C + kTrTile - 1) / kTrTile, (R + kTrTile - 1) / kTrTile);
    const int vec_ok = R % 16 == 0 && C % 16 == 0 && aligned_to(src, 16) && aligned_to(dst, 16);
    transpose_i8_kernel<<<grid, 256, 0, stream>>>(src, dst, R, C, vec_ok);
    return check_launch("transpose_i8_kernel");
}

// Whether the tiled GEMM2 reads the fp16 hidden with on-load quantization
// (gemm_i8_a16_kernel) instead of the int8 hidden.  Both give the same bytes;
// the on-load path was measured slower on MI355X at the BASELINE shape (it
// doubles GEMM2's A bytes and adds ~3 VALU ops per element to a loop that has
// no VALU slack) and needs GEMM1's fp16 hidden, so it also turns off GEMM1's
// fused requantization.  INT8K_MLP_GEMM2_FP16_HIDDEN=1 selects it (read on
// every call and workspace query).
bool gemm2_reads_fp16_hidden() {
    const char* e = std::getenv("INT8K_MLP_GEMM2_FP16_HIDDEN");
    return e != nullptr && e[0] == '1';
}

// Which GEMMs of an MLP call requantize in their epilogue (gemm_i8_rq_kernel):
// those on the 256 x 256 tiled kernel with at most kRqMaxStripeTiles column
// tiles per stripe; GEMM2 only for the per-token output.  The flag
// INT8K_MLP_SEPARATE_REQUANT (or INT8K_MLP_FUSED_REQUANT=0 in the environment,
// read once) keeps both on the fp16 output + requant_rows_kernel path.
struct RqPlan {
    bool g1, g2;
};

inline bool rq_fusable(int M, int N, int K) {
    if (use_skinny(M, N, K) || splitk_plan(M, N, K).use || use_mid(M, N, K)) return false;
    return (N + BN - 1) / BN <= kRqMaxStripeTiles;
}

RqPlan rq_plan(int T, int dm, int dff, int flags) {
    static const bool env_on = [] {
        const char* e = std::getenv("INT8K_MLP_FUSED_REQUANT");
        return !(e != nullptr && e[0] == '0');
    }();
    const bool on = env_on && (flags & INT8K_MLP_SEPARATE_REQUANT) == 0;
    RqPlan pl;
    pl.g1 = on && !gemm2_reads_fp16_hidden() && rq_fusable(T, dff, dm);
    pl.g2 = on && (flags & INT8K_MLP_OUT_PER_TENSOR) == 0 && rq_fusable(T, dm, dff);
    return pl;
}

// Whether a GEMM runs on the 256 x 256 tiled kernels (gemm_i8_kernel, gemm_i8_rq_kernel).
inline bool tiled_256(int M, int N, int K) {
    return !use_skinny(M, N, K) && !splitk_plan(M, N, K).use && !use_mid(M, N, K);
}

// The kernels of one MLP call.  kn1 / kn2: the unpacked weights are read as the
// caller stores them ([K][N]) by the tiled kernels, with no transpose; the other
// tilings (and the fp16-hidden GEMM2) read transposed copies in the workspace.
struct MlpPlan {
    RqPlan rq;
    bool a16;       // GEMM2 reads the fp16 hidden (INT8K_MLP_GEMM2_FP16_HIDDEN=1)
    bool kn1, kn2;
};

MlpPlan mlp_plan(int T, int dm, int dff, int flags) {
    MlpPlan pl;
    pl.rq = rq_plan(T, dm, dff, flags);
    pl.a16 = !pl.rq.g1 && !use_skinny(T, dm, dff) && !splitk_plan(T, dm, dff).use &&
             gemm2_reads_fp16_hidden();
    const bool unpacked = (flags & INT8K_MLP_WEIGHTS_PREPACKED) == 0;
    pl.kn1 = unpacked && tiled_256(T, dff, dm);
    pl.kn2 = unpacked && !pl.a16 && tiled_256(T, dm, dff);
    return pl;
}

// Workspace layout of one MLP call (all offsets 256-byte aligned).
struct MlpWorkspace {
    int8_t* w1t;      // [d_ff][d_model]  (absent when prepacked)
    int8_t* w2t;      // [d_model][d_ff]
    uint16_t* h16;    // [T][d_ff]          (absent when GEMM1 requantizes)
    int8_t* hq;       // [T][d_ff]
    float* sh;        // [T]
    float* p1;        // [tiles_n1][T]      (absent when GEMM1 requantizes)
    uint16_t* o16;    // [T][d_model]       (absent when GEMM2 requantizes)
    float* p2;        // [tiles_n2][T]      (absent when GEMM2 requantizes)
    float* tmax;      // [1]
    uint32_t* sync;   // fused requant: amax1 [T], amax2 [T], arrived1 [tiles_m], arrived2 [tiles_m]
    int sync_words;
    int32_t* part;    // split-K partials (the larger GEMM's), when a GEMM runs split-K
    size_t bytes;
};

MlpWorkspace carve_mlp(void* base, int T, int dm, int dff, bool prepacked, const MlpPlan& pl) {
    const RqPlan& rp = pl.rq;
    char* p = static_cast<char*>(base);
    size_t off = 0;
    auto take = [&](size_t n) {
        char* r = p + off;
        off += round_up(n, kWorkspaceAlign);
        return r;
    };
    MlpWorkspace w{};
    const size_t wbytes = prepacked ? 0 : (size_t)dm * dff;
    w.w1t = reinterpret_cast<int8_t*>(take(pl.kn1 ? 0 : wbytes));
    w.w2t = reinterpret_cast<int8_t*>(take(pl.kn2 ? 0 : wbytes));
    w.h16 = reinterpret_cast<uint16_t*>(take(rp.g1 ? 0 : (size_t)T * dff * 2));
    w.hq = reinterpret_cast<int8_t*>(take((size_t)T * dff));
    w.sh = reinterpret_cast<float*>(take((size_t)T * 4));
    w.p1 = reinterpret_cast<float*>(take(rp.g1 ? 0 : (size_t)epi_tiles(T, dff, dm) * T * 4));
    w.o16 = reinterpret_cast<uint16_t*>(take(rp.g2 ? 0 : (size_t)T * dm * 2));
    w.p2 = reinterpret_cast<float*>(take(rp.g2 ? 0 : (size_t)epi_tiles(T, dm, dff) * T * 4));
    w.tmax = reinterpret_cast<float*>(take(4));
    const int tiles_m = (T + BM - 1) / BM;
    w.sync_words = (rp.g1 || rp.g2) ? 2 * T + 2 * tiles_m : 0;
    w.sync = reinterpret_cast<uint32_t*>(take((size_t)w.sync_words * 4));
    const size_t part1 = use_skinny(T, dff, dm) ? 0 : splitk_partial_bytes(T, dff, dm);
    const size_t part2 = use_skinny(T, dm, dff) ? 0 : splitk_partial_bytes(T, dm, dff);
    w.part = reinterpret_cast<int32_t*>(take(std::max(part1, part2)));
    w.bytes = off;
    return w;
}

PerDeviceOnce lds_once;

int configure_lds() {
    return lds_once.run([] {
        hipError_t e = hipFuncSetAttribute((const void*)gemm_i8_kernel<EPI_I32>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)gemm_i8_kernel<EPI_GELU_F16>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kEpiLdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)gemm_i8_kernel<EPI_F16>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kEpiLdsBytes);
        const void* epi_kernels[] = {
            (const void*)gemm_i8_rq_kernel<EPI_GELU_F16>, (const void*)gemm_i8_rq_kernel<EPI_F16>,
            (const void*)gemm_i8_rq_kernel<EPI_GELU_F16, true>,
            (const void*)gemm_i8_rq_kernel<EPI_F16, true>,
            (const void*)gemm_i8_kernel<EPI_GELU_F16, true>, (const void*)gemm_i8_kernel<EPI_F16, true>};
        for (const void* k : epi_kernels)
            if (e == hipSuccess)
                e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kEpiLdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)gemm_i8_a16_kernel,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kA16LdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)gemm_i8_mid_kernel<EPI_GELU_F16>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kMidEpiLds);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)gemm_i8_mid_kernel<EPI_F16>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kMidEpiLds);
        if (e != hipSuccess) {
            set_last_error("hipFuncSetAttribute", e);
            return (int)INT8K_ERR_HIP;
        }
        return (int)INT8K_OK;
    });
}

}  // namespace
}  // namespace int8k

using namespace int8k;

extern "C" int int8k_gemm_i8_i32(const int8_t* A, const int8_t* Bt, int32_t* C, int M, int N,
                                 int K, void* stream) {
    clear_last_error();
    if (!A || !Bt || !C || M <= 0 || N <= 0 || K <= 0) return INT8K_ERR_INVALID_ARGUMENT;
    if (K % 16 != 0) return INT8K_ERR_UNSUPPORTED;
    if (!aligned_to(A, 16) || !aligned_to(Bt, 16) || !aligned_to(C, 4)) return INT8K_ERR_MISALIGNED;
    if (int st = check_tiled_operands(M, N, K)) return st;
    int st = configure_lds();
    if (st != INT8K_OK) return st;
    EpiParams p{};
    p.c32 = C;
    p.ldc = N;
    return launch_gemm<EPI_I32>(A, Bt, M, N, K, p, as_stream(stream));
}

extern "C" int int8k_transpose_int8_weights(const int8_t* W1, const int8_t* W2, int8_t* W1T,
                                            int8_t* W2T, int d_model, int d_ff, void* stream) {
    clear_last_error();
    if (!W1 || !W2 || !W1T || !W2T || d_model <= 0 || d_ff <= 0) return INT8K_ERR_INVALID_ARGUMENT;
    int st = launch_transpose(W1, W1T, d_model, d_ff, as_stream(stream));
    if (st != INT8K_OK) return st;
    return launch_transpose(W2, W2T, d_ff, d_model, as_stream(stream));
}

extern "C" size_t int8k_mlp_workspace_bytes(int T, int d_model, int d_ff, int flags) {
    if (T <= 0 || d_model <= 0 || d_ff <= 0) return 0;
    return carve_mlp(nullptr, T, d_model, d_ff, (flags & INT8K_MLP_WEIGHTS_PREPACKED) != 0,
                     mlp_plan(T, d_model, d_ff, flags))
        .bytes;
}

extern "C" int int8k_mlp_sync_timeouts(unsigned int* count) {
    clear_last_error();
    if (!count) return INT8K_ERR_INVALID_ARGUMENT;
    const hipError_t e = hipMemcpyFromSymbol(count, HIP_SYMBOL(g_rq_timeouts), sizeof(unsigned int),
                                             0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        set_last_error("hipMemcpyFromSymbol(g_rq_timeouts)", e);
        return INT8K_ERR_HIP;
    }
    return INT8K_OK;
}

extern "C" int int8k_mlp_forward(const int8_t* x, const int8_t* W1, const int8_t* W2, int8_t* out,
                                 const float* scale_x, int n_scale_x, const float* scale_W1,
                                 int n_scale_W1, const float* scale_W2, int n_scale_W2,
                                 const float* bias1, float* out_scale, int T, int d_model,
                                 int d_ff, int flags, void* workspace, size_t workspace_bytes,
                                 void* stream) {
    clear_last_error();
    if (!x || !W1 || !W2 || !out || !scale_x || !scale_W1 || !scale_W2 || !out_scale)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (T <= 0 || d_model <= 0 || d_ff <= 0) return INT8K_ERR_INVALID_ARGUMENT;
    if ((n_scale_x != 1 && n_scale_x != T) || (n_scale_W1 != 1 && n_scale_W1 != d_ff) ||
        (n_scale_W2 != 1 && n_scale_W2 != d_model))
        return INT8K_ERR_INVALID_ARGUMENT;
    if ((flags & ~(INT8K_MLP_WEIGHTS_PREPACKED | INT8K_MLP_OUT_PER_TENSOR |
                   INT8K_MLP_SEPARATE_REQUANT)) != 0)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (d_model % 16 != 0 || d_ff % 16 != 0) return INT8K_ERR_UNSUPPORTED;
    if (!aligned_to(x, 16) || !aligned_to(W1, 16) || !aligned_to(W2, 16) || !aligned_to(out, 4) ||
        !aligned_to(scale_x, 4) || !aligned_to(scale_W1, 4) || !aligned_to(scale_W2, 4) ||
        !aligned_to(out_scale, 4) || (bias1 && !aligned_to(bias1, 4)))
        return INT8K_ERR_MISALIGNED;
    const bool prepacked = (flags & INT8K_MLP_WEIGHTS_PREPACKED) != 0;
    const bool per_tensor_out = (flags & INT8K_MLP_OUT_PER_TENSOR) != 0;
    const MlpPlan pl = mlp_plan(T, d_model, d_ff, flags);
    const RqPlan& rp = pl.rq;
    // operands of 4 GiB or more on a 256 x 256 GEMM: refused before anything is launched
    if (tiled_256(T, d_ff, d_model))
        if (int st = check_tiled_operands(T, d_ff, d_model)) return st;
    if (tiled_256(T, d_model, d_ff) && !pl.a16)
        if (int st = check_tiled_operands(T, d_model, d_ff)) return st;
    const MlpWorkspace w = carve_mlp(workspace, T, d_model, d_ff, prepacked, pl);
    if (!workspace || workspace_bytes < w.bytes) return INT8K_ERR_WORKSPACE;
    if (!aligned_to(workspace, 256)) return INT8K_ERR_MISALIGNED;
    int st = configure_lds();
    if (st != INT8K_OK) return st;
    hipStream_t s = as_stream(stream);
    const int tiles_m = (T + BM - 1) / BM;
    uint32_t* amax1 = w.sync;
    uint32_t* amax2 = w.sync + T;
    uint32_t* arrived1 = w.sync + 2 * T;
    uint32_t* arrived2 = arrived1 + tiles_m;
    if (w.sync_words > 0) {
        rq_clear_kernel<<<std::min(64, (w.sync_words + 255) / 256), 256, 0, s>>>(w.sync,
                                                                               w.sync_words);
        if ((st = check_launch("rq_clear_kernel")) != INT8K_OK) return st;
    }

    // W1t / W2t: [N][K] operands (prepacked, or transposed here), or the caller's
    // [K][N] weights themselves where kn1 / kn2 read them as stored
    const int8_t* W1t = W1;
    const int8_t* W2t = W2;
    if (!prepacked && !pl.kn1) {
        if ((st = launch_transpose(W1, w.w1t, d_model, d_ff, s)) != INT8K_OK) return st;
        W1t = w.w1t;
    }
    if (!prepacked && !pl.kn2) {
        if ((st = launch_transpose(W2, w.w2t, d_ff, d_model, s)) != INT8K_OK) return st;
        W2t = w.w2t;
    }
    // GEMM1 + scale/bias/GELU epilogue -> int8 hidden + row scales (fused requant), or
    // fp16 hidden + row absmax partials for the separate pass
    EpiParams p1{};
    p1.c16 = w.h16;
    p1.ldc = d_ff;
    p1.sa = scale_x;
    p1.sa_stride = n_scale_x == 1 ? 0 : 1;
    p1.sb = scale_W1;
    p1.sb_stride = n_scale_W1 == 1 ? 0 : 1;
    p1.bias = bias1;
    p1.pmax = w.p1;
    const SplitKPlan sk1 = splitk_plan(T, d_ff, d_model);
    if (rp.g1 && pl.kn1)
        st = launch_gemm_rq<EPI_GELU_F16, true>(x, W1t, T, d_ff, d_model, p1, w.hq, w.sh, amax1,
                                                arrived1, s);
    else if (rp.g1)
        st = launch_gemm_rq<EPI_GELU_F16>(x, W1t, T, d_ff, d_model, p1, w.hq, w.sh, amax1,
                                          arrived1, s);
    else if (pl.kn1)
        st = launch_gemm<EPI_GELU_F16, true>(x, W1t, T, d_ff, d_model, p1, s);
    else if (use_skinny(T, d_ff, d_model))
        st = launch_gemm_skinny<EPI_GELU_F16>(x, W1t, T, d_ff, d_model, p1, s);
    else if (sk1.use)
        st = launch_gemm_splitk<EPI_GELU_F16>(x, W1t, T, d_ff, d_model, sk1, w.part, p1, s);
    else if (use_mid(T, d_ff, d_model))
        st = launch_gemm_mid<EPI_GELU_F16>(x, W1t, T, d_ff, d_model, p1, s);
    else
        st = launch_gemm<EPI_GELU_F16>(x, W1t, T, d_ff, d_model, p1, s);
    if (st != INT8K_OK) return st;
    // GEMM2 + dequant epilogue -> int8 output + scales (fused requant), or fp16 output +
    // absmax partials for the separate pass
    const int tn1 = epi_tiles(T, d_ff, d_model);
    EpiParams p2{};
    p2.c16 = w.o16;
    p2.ldc = d_model;
    p2.sa = w.sh;
    p2.sa_stride = 1;
    p2.sb = scale_W2;
    p2.sb_stride = n_scale_W2 == 1 ? 0 : 1;
    p2.pmax = w.p2;
    const SplitKPlan sk2 = splitk_plan(T, d_model, d_ff);
    const bool skinny2 = use_skinny(T, d_model, d_ff);
    // the on-load path has 256 x 256 tiles on every grid it runs
    const bool a16 = pl.a16;
    if (!rp.g1 && !a16) {
        // per-token requant of the hidden (one absmax partial per row and 256-column
        // tile, or per 32-column block of the skinny path)
        if ((st = launch_requant(w.h16, d_ff, w.p1, tn1, nullptr, w.hq, d_ff, w.sh, T, d_ff,
                                 s)) != INT8K_OK)
            return st;
    }
    if (rp.g2 && pl.kn2)
        return launch_gemm_rq<EPI_F16, true>(w.hq, W2t, T, d_model, d_ff, p2, out, out_scale,
                                             amax2, arrived2, s);
    if (rp.g2)
        return launch_gemm_rq<EPI_F16>(w.hq, W2t, T, d_model, d_ff, p2, out, out_scale, amax2,
                                       arrived2, s);
    if (a16) {
        // the tiled GEMM2 reads the fp16 hidden and quantizes it per row on load
        const int tiles_m = (T + BM - 1) / BM, tiles_n = (d_model + BN - 1) / BN;
        gemm_i8_a16_kernel<<<tiles_m * tiles_n, kThreads, kA16LdsBytes, s>>>(
            w.h16, W2t, T, d_model, d_ff, tiles_m, tiles_n, w.p1, tn1, p2);
        if ((st = check_launch("gemm_i8_a16_kernel")) != INT8K_OK) return st;
    } else {
        if (pl.kn2)
            st = launch_gemm<EPI_F16, true>(w.hq, W2t, T, d_model, d_ff, p2, s);
        else if (skinny2)
            st = launch_gemm_skinny<EPI_F16>(w.hq, W2t, T, d_model, d_ff, p2, s);
        else if (sk2.use)
            st = launch_gemm_splitk<EPI_F16>(w.hq, W2t, T, d_model, d_ff, sk2, w.part, p2, s);
        else if (use_mid(T, d_model, d_ff))
            st = launch_gemm_mid<EPI_F16>(w.hq, W2t, T, d_model, d_ff, p2, s);
        else
            st = launch_gemm<EPI_F16>(w.hq, W2t, T, d_model, d_ff, p2, s);
        if (st != INT8K_OK) return st;
    }
    const int tn2 = a16 ? (d_model + BN - 1) / BN : epi_tiles(T, d_model, d_ff);
    const float* tmax = nullptr;
    if (per_tensor_out) {
        tensor_absmax_kernel<<<1, 256, 0, s>>>(w.p2, (size_t)tn2 * T, w.tmax);
        if ((st = check_launch("tensor_absmax_kernel")) != INT8K_OK) return st;
        tmax = w.tmax;
    }
    return launch_requant(w.o16, d_model, w.p2, tn2, tmax, out, d_model, out_scale, T, d_model,
                          s);
}
