// gemm_i8.h — int8 x int8 -> int32 GEMM core on gfx950 MFMA, with fused epilogues.
//
//   C[M,N] = A[M,K] . Bt[N,K]^T      (both operands K-contiguous, row-major)
//
// Block tile 256 x 256 x 128, 256 threads = 4 waves in a 2 x 2 grid, each wave
// owning a 128 x 128 sub-tile as 4 x 4 v_mfma_i32_32x32x32_i8 accumulators
// (256 accumulator registers per lane).  Operands are staged global -> VGPR ->
// LDS (double-buffered, rows padded to 144 bytes so the 16-byte fragment
// reads of consecutive rows spread over the banks); the next K-step's global loads are
// in flight while the current one runs on the matrix cores.  Blocks are mapped
// XCD-first (consecutive tiles share an XCD and its L2) and grouped along M.
//
// Internal header of libint8k (mlp.hip, prefill.hip).
#pragma once

#include "int8k_common.h"

namespace int8k {
namespace gemm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int kThreads = 256;
constexpr int WM = 128, WN = 128;           // wave tile
constexpr int TM = WM / 32, TN = WN / 32;   // 32x32 MFMA tiles per wave
constexpr int LDS_STRIDE = BK + 16;         // padded row, bytes
constexpr int A_STAGE = BM * LDS_STRIDE;
constexpr int B_STAGE = BN * LDS_STRIDE;
constexpr int STAGE_BYTES = A_STAGE + B_STAGE;
constexpr int LDS_BYTES = 2 * STAGE_BYTES;  // 147456 of gfx950's 160 KiB
constexpr int kChunksPerRow = BK / 16;
constexpr int kChunks = BM * kChunksPerRow / kThreads;  // 16-byte chunks per thread per operand
constexpr int kNumXcd = 8;
constexpr int kGroupM = 8;

// Linear block id -> (tile_m, tile_n): XCD-contiguous ranges, grouped along M.
__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    const int xcd = bid % kNumXcd;
    const int local = bid / kNumXcd;
    const int base = total / kNumXcd, rem = total % kNumXcd;
    const int tile = xcd * base + min(xcd, rem) + local;
    const int per_group = kGroupM * tiles_n;
    const int group = tile / per_group;
    const int first_m = group * kGroupM;
    const int gm = min(tiles_m - first_m, kGroupM);
    const int in_group = tile - group * per_group;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

struct Frag {
    int4 a[kChunks];
    int4 b[kChunks];
};

// Global -> registers for one K-step.  Chunk c (16 B) of a 256 x BK operand
// tile: row c / (BK/16), bytes (c % (BK/16)) * 16.  Rows past the matrix and
// K past the end read a clamped in-bounds address; store_stage zeroes them,
// so the loads themselves are unconditional and their wait lands late.
__device__ __forceinline__ void load_stage(Frag& f, const int8_t* __restrict__ A,
                                           const int8_t* __restrict__ Bt, int M, int N, int K,
                                           int lda, int ldb, int m0, int n0, int k0) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = t + i * kThreads;
        const int row = c / kChunksPerRow, kc = (c % kChunksPerRow) * 16;
        const int gk = min(k0 + kc, K - 16);
        f.a[i] = *reinterpret_cast<const int4*>(A + (size_t)min(m0 + row, M - 1) * lda + gk);
        f.b[i] = *reinterpret_cast<const int4*>(Bt + (size_t)min(n0 + row, N - 1) * ldb + gk);
    }
}

// One chunk of each operand (index i of load_stage) — for interleaving.
__device__ __forceinline__ int4 load_chunk(const int8_t* __restrict__ P, int rows, int K, int ld,
                                           int r0, int k0, int i) {
    const int c = threadIdx.x + i * kThreads;
    const int row = c / kChunksPerRow, kc = (c % kChunksPerRow) * 16;
    const int gk = min(k0 + kc, K - 16);
    return *reinterpret_cast<const int4*>(P + (size_t)min(r0 + row, rows - 1) * ld + gk);
}

template <bool EDGE>
__device__ __forceinline__ void store_chunk(int4 v, char* lds_op, int rows, int K, int r0, int k0,
                                            int i) {
    const int c = threadIdx.x + i * kThreads;
    const int row = c / kChunksPerRow, kc = (c % kChunksPerRow) * 16;
    if constexpr (EDGE) {
        if (!(k0 + kc < K && r0 + row < rows)) v = make_int4(0, 0, 0, 0);
    }
    *reinterpret_cast<int4*>(lds_op + row * LDS_STRIDE + kc) = v;
}

__device__ __forceinline__ v4i read_frag(const char* stage, int off, int t, int slice) {
    return *reinterpret_cast<const v4i*>(stage + off + t * 32 * LDS_STRIDE + slice * 32);
}

// Registers -> LDS.  EDGE zeroes the chunks that load_stage clamped.
template <bool EDGE>
__device__ __forceinline__ void store_stage(const Frag& f, char* lds, int M, int N, int K,
                                            int m0, int n0, int k0) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = t + i * kThreads;
        const int row = c / kChunksPerRow, kc = (c % kChunksPerRow) * 16;
        int4 va = f.a[i], vb = f.b[i];
        if constexpr (EDGE) {
            const bool kok = k0 + kc < K;
            if (!(kok && m0 + row < M)) va = make_int4(0, 0, 0, 0);
            if (!(kok && n0 + row < N)) vb = make_int4(0, 0, 0, 0);
        }
        *reinterpret_cast<int4*>(lds + row * LDS_STRIDE + kc) = va;
        *reinterpret_cast<int4*>(lds + A_STAGE + row * LDS_STRIDE + kc) = vb;
    }
}

__device__ __forceinline__ void read_slice(v4i (&a)[TM], v4i (&b)[TN], const char* stage,
                                           int a_off, int b_off, int slice) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
        a[i] = *reinterpret_cast<const v4i*>(stage + a_off + i * 32 * LDS_STRIDE + slice * 32);
#pragma unroll
    for (int j = 0; j < TN; ++j)
        b[j] = *reinterpret_cast<const v4i*>(stage + b_off + j * 32 * LDS_STRIDE + slice * 32);
}

// One 32x32x32 MFMA of tile (i, j).  SWAP computes the tile transposed (B . A^T):
// the same sums, with a lane holding one row and 16 columns instead of one
// column and 16 rows (see acc_row).
template <bool SWAP>
__device__ __forceinline__ v16i mfma_ab(const v4i& a, const v4i& b, const v16i& c) {
    if constexpr (SWAP) return __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <bool SWAP = false>
__device__ __forceinline__ void mfma_slice(v16i (&acc)[TM][TN], const v4i (&a)[TM],
                                           const v4i (&b)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
            acc[i][j] = mfma_ab<SWAP>(a[i], b[j], acc[i][j]);
}

// ------------------------------------------------------------ B stored [K][N]
// The MLP's weights as the caller holds them (W1 [d_model][d_ff], W2 [d_ff][d_model])
// are N-contiguous.  With BKN the main loop stages the B tile as it arrives, BK
// rows of k with the tile's BN bytes of n each (rows padded to KN_STRIDE), and
// forms each K-contiguous MFMA fragment with two transposing LDS reads
// (ds_read_b64_tr_b8), so no weight transpose runs.  Measured on the box: in each
// group of 16 lanes, the instruction gives lane 8h + b byte b of the 8-byte rows
// that lanes h, h+2, ..., h+14 address.  Lane s of group g therefore addresses
// row 16 (g/2) + s/2 at columns 16 (g%2) + 8 (s%2): lane l then holds
// k = 16 (l/32) + 0..7 of column l % 32, the B fragment's layout, and a second
// read 8 rows further gives k + 8..15.
constexpr int KN_STRIDE = BN + 32;  // 288 B: the 16 rows of one read start 32 B apart in the banks
static_assert(BK * KN_STRIDE == B_STAGE, "the [K][N] B tile takes the stage bytes of [N][K]");

// Chunk i of this thread of a [K][N] B tile: k row c / 16, n bytes (c % 16) * 16
// (16 threads per 256-byte row).  N % 16 == 0; chunks past K or N read a clamped
// address and are zeroed when stored (EDGE).
__device__ __forceinline__ int4 load_chunk_kn(const int8_t* __restrict__ W, int K, int N, int ldw,
                                              int k0, int n0, int i) {
    const int c = threadIdx.x + i * kThreads;
    const int kr = c >> 4, nc = (c & 15) * 16;
    return *reinterpret_cast<const int4*>(W + (size_t)min(k0 + kr, K - 1) * ldw +
                                          min(n0 + nc, N - 16));
}

template <bool EDGE>
__device__ __forceinline__ void store_chunk_kn(int4 v, char* lds_b, int K, int N, int k0, int n0,
                                               int i) {
    const int c = threadIdx.x + i * kThreads;
    const int kr = c >> 4, nc = (c & 15) * 16;
    if constexpr (EDGE) {
        if (!(k0 + kr < K && n0 + nc < N)) v = make_int4(0, 0, 0, 0);
    }
    *reinterpret_cast<int4*>(lds_b + kr * KN_STRIDE + nc) = v;
}

// This lane's address inside a [K][N] B stage for fragment reads (see above).
__device__ __forceinline__ int kn_frag_offset(int lane, int wn) {
    const int g = lane >> 4, s = lane & 15;
    return (16 * (g >> 1) + (s >> 1)) * KN_STRIDE + wn * WN + 16 * (g & 1) + 8 * (s & 1);
}

// B fragment of column tile j, k-slice `slice`, from a [K][N] stage.
__device__ __forceinline__ v4i read_frag_kn(const char* stage_b, int off, int j, int slice) {
    typedef int v2i __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) v2i lds_v2i;
    const char* p = stage_b + off + slice * 32 * KN_STRIDE + j * 32;
    const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(p));
    const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(p + 8 * KN_STRIDE));
    return v4i{lo.x, lo.y, hi.x, hi.y};
}

// Instruction classes for __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedVmemRead = 0x020, kSchedDsRead = 0x100,
              kSchedDsWrite = 0x200;

// NR LDS reads interleaved with the first NR of 16 MFMAs.
template <int NR = 8>
__device__ __forceinline__ void sched_reads_mfma() {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 16 - NR, 0);
}

// Main-loop operand loads through buffer resources: one 32-bit offset per
// thread and operand, the chunk index and the K-step adding uniform (scalar)
// offsets, so a load needs no per-chunk address arithmetic.  The resource
// covers exactly the operand's bytes ((rows - 1) * ld + cols): rows past the
// matrix read as zero, and chunks past K (N for a [K][N] B) inside a row are
// zeroed when stored (EDGE), as with the clamped loads above.
struct OperandSrc {
    __amdgpu_buffer_rsrc_t r;
    uint32_t voff;        // this thread's chunk 0 at K-step 0
    uint32_t chunk_step;  // bytes between chunks i and i+1 of a thread
    uint32_t k_mul;       // bytes per unit of k0 (1 for K-contiguous, ld for [K][N])
};

// [rows][ld] K-contiguous operand, tile rows r0 ..: thread t's chunk i is row
// t/8 + 32 i, bytes (t%8)*16 of the K-step.
__device__ __forceinline__ OperandSrc operand_rowmajor(const int8_t* P, int rows, int cols, int ld,
                                                       int r0) {
    OperandSrc s;
    s.r = make_buffer(P, (uint32_t)((size_t)(rows - 1) * ld + cols));
    const int t = threadIdx.x;
    s.voff = (uint32_t)(r0 + t / kChunksPerRow) * (uint32_t)ld + (t % kChunksPerRow) * 16;
    s.chunk_step = (uint32_t)(kThreads / kChunksPerRow) * (uint32_t)ld;
    s.k_mul = 1;
    return s;
}

// [K][ldw] N-contiguous B, tile columns n0 ..: thread t's chunk i is k row
// t/16 + 16 i, bytes (t%16)*16 of the tile's 256 columns.
__device__ __forceinline__ OperandSrc operand_kn(const int8_t* W, int K, int N, int ldw, int n0) {
    OperandSrc s;
    s.r = make_buffer(W, (uint32_t)((size_t)(K - 1) * ldw + N));
    const int t = threadIdx.x;
    s.voff = (uint32_t)(t >> 4) * (uint32_t)ldw + (uint32_t)n0 + (t & 15) * 16;
    s.chunk_step = (uint32_t)(kThreads / 16) * (uint32_t)ldw;
    s.k_mul = (uint32_t)ldw;
    return s;
}

__device__ __forceinline__ int4 load_operand(const OperandSrc& s, int k0, int i) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const v4u w = __builtin_amdgcn_raw_buffer_load_b128(
        s.r, s.voff, (uint32_t)k0 * s.k_mul + (uint32_t)i * s.chunk_step, 0);
    return make_int4((int)w.x, (int)w.y, (int)w.z, (int)w.w);
}

// The MFMA main loop: acc[i][j] (32x32 tiles) of this wave's 128x128 sub-tile.
//
// With one wave per SIMD the wave stalls on every MFMA issue, so all other
// work of a K-step is threaded between MFMAs (sched_group_barrier) instead of
// being issued in bursts.  K-step kt computes on LDS buffer kt&1 in four
// 32-wide k slices:
//   slices 0, 1: LDS reads of slice s+1 between the MFMAs of slice s
//   slice 2:     LDS reads of slice 3, the LDS writes of stage kt+1 (held in
//                registers since step kt-1) and the global loads of stage
//                kt+2, all between the MFMAs of slice 2
//   slice 3:     8 MFMAs, the barrier, then the LDS reads of slice 0 of
//                stage kt+1 between the last 8 MFMAs
// Writing buffer (kt+1)&1 during step kt is safe: its last reads (step kt-1)
// completed before step kt-1's barrier.  Past the end of K the loads clamp to
// valid addresses and the writes land in the buffer nobody reads again.
// BKN: Bt is B stored [K][N] (row stride ldb), staged and read as above.
template <bool EDGE, bool SWAP = false, bool BKN = false>
__device__ __forceinline__ void mainloop(v16i (&acc)[TM][TN], const int8_t* __restrict__ A,
                                         const int8_t* __restrict__ Bt, int M, int N, int K,
                                         int lda, int ldb, int m0, int n0, char* lds) {
    static_assert(BK == 128, "the schedule below is written for 4 k-slices per stage");
    static_assert(kChunks == 8, "the schedule below threads 16 loads and writes per step");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    const int nk = (K + BK - 1) / BK;
    // fragment read offsets inside a stage: row (l%32), 16-byte half (l/32)
    const int a_off = (wm * WM + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 16;
    const int b_off = BKN ? kn_frag_offset(lane, wn)
                          : A_STAGE + (wn * WN + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 16;
    const OperandSrc srcA = operand_rowmajor(A, M, K, lda, m0);
    const OperandSrc srcB = BKN ? operand_kn(Bt, K, N, ldb, n0) : operand_rowmajor(Bt, N, K, ldb, n0);
    auto load_a = [&](int k0, int i) { return load_operand(srcA, k0, i); };
    auto load_b = [&](int k0, int i) { return load_operand(srcB, k0, i); };
    auto store_b = [&](int4 v, char* stage, int k0, int i) {
        if constexpr (BKN) store_chunk_kn<EDGE>(v, stage + A_STAGE, K, N, k0, n0, i);
        else store_chunk<EDGE>(v, stage + A_STAGE, N, K, n0, k0, i);
    };
    auto read_b = [&](const char* stage, int j, int slice) {
        return BKN ? read_frag_kn(stage + A_STAGE, b_off, j, slice)
                   : read_frag(stage, b_off, j, slice);
    };
    auto read_ab = [&](v4i (&a)[TM], v4i (&b)[TN], const char* stage, int slice) {
#pragma unroll
        for (int i = 0; i < TM; ++i) a[i] = read_frag(stage, a_off, i, slice);
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = read_b(stage, j, slice);
    };
    constexpr int kReads = BKN ? TM + 2 * TN : TM + TN;  // LDS read instructions per slice
    Frag f;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        f.a[i] = load_a(0, i);
        f.b[i] = load_b(0, i);
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        store_chunk<EDGE>(f.a[i], lds, M, K, m0, 0, i);
        store_b(f.b[i], lds, 0, i);
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        f.a[i] = load_a(BK, i);
        f.b[i] = load_b(BK, i);
    }
    __syncthreads();
    v4i a[2][TM], b[2][TN];
    read_ab(a[0], b[0], lds, 0);
    for (int kt = 0; kt < nk; ++kt) {
        const char* cur = lds + (kt & 1) * STAGE_BYTES;
        char* nxt = lds + ((kt + 1) & 1) * STAGE_BYTES;
        __builtin_amdgcn_sched_barrier(0);
        read_ab(a[1], b[1], cur, 1);
        mfma_slice<SWAP>(acc, a[0], b[0]);
        sched_reads_mfma<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        read_ab(a[0], b[0], cur, 2);
        mfma_slice<SWAP>(acc, a[1], b[1]);
        sched_reads_mfma<kReads>();
        __builtin_amdgcn_sched_barrier(0);
        // slice 2, one group per MFMA: a fragment read of slice 3, a chunk
        // written to the next stage and its replacement load, then the MFMA
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const int i = g >> 2, j = g & 3;
            if (g < 4) a[1][g] = read_frag(cur, a_off, g, 3);
            else if (g < 8) b[1][g - 4] = read_b(cur, g - 4, 3);
            if (g < 8) {
                store_chunk<EDGE>(f.a[g], nxt, M, K, m0, (kt + 1) * BK, g);
                f.a[g] = load_a((kt + 2) * BK, g);
            } else {
                store_b(f.b[g - 8], nxt, (kt + 1) * BK, g - 8);
                f.b[g - 8] = load_b((kt + 2) * BK, g - 8);
            }
            acc[i][j] = mfma_ab<SWAP>(a[0][i], b[0][j], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // slice 3: half of its MFMAs cover the LDS writes before the barrier,
        // the other half the reads of the next stage's slice 0 after it
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            acc[g >> 2][g & 3] = mfma_ab<SWAP>(a[1][g >> 2], b[1][g & 3], acc[g >> 2][g & 3]);
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
#pragma unroll
        for (int g = 8; g < 16; ++g) {
            if (g < 12) a[0][g - 8] = read_frag(nxt, a_off, g - 8, 0);
            else b[0][g - 12] = read_b(nxt, g - 12, 0);
            acc[g >> 2][g & 3] = mfma_ab<SWAP>(a[1][g >> 2], b[1][g & 3], acc[g >> 2][g & 3]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// ------------------------------------------------------------ fp16 A operand
// The MLP's second GEMM can read the fp16 hidden h [M][K] itself and quantize
// it per row on its way to LDS: code = rint(clamp(h * inv_row, -128, 127)),
// inv_row = 127 / amax_row, the codes of the separate requantization pass
// (requant_rows_kernel) for every finite h.  Each thread's 8 A chunks lie on
// 8 fixed rows (c / 8 for chunk c), so their inv sit in registers.

// rint(fl(h * inv)) of the 16 fp16 of a chunk as 16 packed int8.  fl(h * inv)
// is one v_fma_mix_f32 with a +0 addend (one rounding, as the pass's
// multiply; the sign of a zero product does not reach the code).  Adding
// 1.5 * 2^23 rounds half to even onto the integer grid and leaves the code in
// the low byte of the sum's bits for |h * inv| < 2^22; |h| <= amax (1 + 2^-11)
// keeps |h * inv| below 127.5, so no clamp is needed.  EXACT (a block with a
// row max above the fp16 range, whose h may be infinite) clamps first, as the
// pass does.
template <bool EXACT>
__device__ __forceinline__ int4 quant_chunk_f16(const uint4 (&h)[2], float inv) {
#pragma clang fp contract(off)
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t w[8] = {h[0].x, h[0].y, h[0].z, h[0].w, h[1].x, h[1].y, h[1].z, h[1].w};
    uint32_t t[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const h2 v = __builtin_bit_cast(h2, w[j]);
        float p0 = __builtin_fmaf((float)v.x, inv, 0.0f);
        float p1 = __builtin_fmaf((float)v.y, inv, 0.0f);
        if constexpr (EXACT) {
            p0 = fminf(fmaxf(p0, -128.f), 127.f);
            p1 = fminf(fmaxf(p1, -128.f), 127.f);
        }
        t[2 * j] = __float_as_uint(p0 + 12582912.0f);
        t[2 * j + 1] = __float_as_uint(p1 + 12582912.0f);
    }
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        o[q] = __builtin_amdgcn_perm(t[4 * q + 1], t[4 * q], 0x0c0c0400u) |
               __builtin_amdgcn_perm(t[4 * q + 3], t[4 * q + 2], 0x04000c0cu);
    return make_int4((int)o[0], (int)o[1], (int)o[2], (int)o[3]);
}

// Chunk i of this thread (16 elements of row (t + 256 i) / 8): the 32 bytes of
// fp16, clamped in bounds like load_chunk.
__device__ __forceinline__ void load_chunk_f16(uint4 (&dst)[2], const uint16_t* __restrict__ A16,
                                               int rows, int K, int ld, int r0, int k0, int i) {
    const int c = threadIdx.x + i * kThreads;
    const int row = c / kChunksPerRow, kc = (c % kChunksPerRow) * 16;
    const int gk = min(k0 + kc, K - 16);
    const uint4* p = reinterpret_cast<const uint4*>(A16 + (size_t)min(r0 + row, rows - 1) * ld + gk);
    dst[0] = p[0];
    dst[1] = p[1];
}

constexpr int kSchedValu = 0x002;

// mainloop with an fp16 A: the same schedule, plus the conversion of the next
// stage's A chunks (loaded a whole K-step earlier) threaded between the MFMAs
// of slices 0 and 1 (chunks 0-3 and 4-7), so slice 2 only stores the codes.
// inv[i]: the row scale of chunk i's row.
template <bool EDGE, bool EXACT>
__device__ __forceinline__ void mainloop_a16(v16i (&acc)[TM][TN], const uint16_t* __restrict__ A16,
                                             const int8_t* __restrict__ Bt, int M, int N, int K,
                                             int lda, int ldb, int m0, int n0, char* lds,
                                             const float (&inv)[kChunks]) {
    static_assert(BK == 128 && kChunks == 8, "schedule written for 4 k-slices and 8 chunks");
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

    const int nk = (K + BK - 1) / BK;
    const int a_off = (wm * WM + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 16;
    const int b_off = A_STAGE + (wn * WN + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 16;
    uint4 ar[kChunks][2];  // raw fp16 A of the stage after next
    int4 aq[kChunks];      // codes of the next stage's A
    int4 br[kChunks];
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        load_chunk_f16(ar[i], A16, M, K, lda, m0, 0, i);
        br[i] = load_chunk(Bt, N, K, ldb, n0, 0, i);
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        store_chunk<EDGE>(quant_chunk_f16<EXACT>(ar[i], inv[i]), lds, M, K, m0, 0, i);
        store_chunk<EDGE>(br[i], lds + A_STAGE, N, K, n0, 0, i);
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        load_chunk_f16(ar[i], A16, M, K, lda, m0, BK, i);
        br[i] = load_chunk(Bt, N, K, ldb, n0, BK, i);
    }
    __syncthreads();
    v4i a[2][TM], b[2][TN];
    read_slice(a[0], b[0], lds, a_off, b_off, 0);
    for (int kt = 0; kt < nk; ++kt) {
        const char* cur = lds + (kt & 1) * STAGE_BYTES;
        char* nxt = lds + ((kt + 1) & 1) * STAGE_BYTES;
        __builtin_amdgcn_sched_barrier(0);
        // slice 0: reads of slice 1, conversion of chunks 0-3
        read_slice(a[1], b[1], cur, a_off, b_off, 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) aq[i] = quant_chunk_f16<EXACT>(ar[i], inv[i]);
        mfma_slice(acc, a[0], b[0]);
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            if (g < 8) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedValu, 11, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        // slice 1: reads of slice 2, conversion of chunks 4-7
        read_slice(a[0], b[0], cur, a_off, b_off, 2);
#pragma unroll
        for (int i = 4; i < 8; ++i) aq[i] = quant_chunk_f16<EXACT>(ar[i], inv[i]);
        mfma_slice(acc, a[1], b[1]);
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            if (g < 8) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedValu, 11, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        // slice 2: reads of slice 3, the next stage's stores, the loads of the one after
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            const int i = g >> 2, j = g & 3;
            if (g < 4) a[1][g] = read_frag(cur, a_off, g, 3);
            else if (g < 8) b[1][g - 4] = read_frag(cur, b_off, g - 4, 3);
            if (g < 8) {
                store_chunk<EDGE>(aq[g], nxt, M, K, m0, (kt + 1) * BK, g);
                load_chunk_f16(ar[g], A16, M, K, lda, m0, (kt + 2) * BK, g);
            } else {
                store_chunk<EDGE>(br[g - 8], nxt + A_STAGE, N, K, n0, (kt + 1) * BK, g - 8);
                br[g - 8] = load_chunk(Bt, N, K, ldb, n0, (kt + 2) * BK, g - 8);
            }
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[0][i], b[0][j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            acc[g >> 2][g & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                a[1][g >> 2], b[1][g & 3], acc[g >> 2][g & 3], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
#pragma unroll
        for (int g = 8; g < 16; ++g) {
            if (g < 12) a[0][g - 8] = read_frag(nxt, a_off, g - 8, 0);
            else b[0][g - 12] = read_frag(nxt, b_off, g - 12, 0);
            acc[g >> 2][g & 3] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                a[1][g >> 2], b[1][g & 3], acc[g >> 2][g & 3], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Accumulator element r of a 32x32 MFMA tile held by `lane`:
//   row = (r/4)*8 + (lane/32)*4 + r%4,  col = lane%32.
// With SWAP the roles trade: row = lane%32, col = acc_row(r, lane).
__device__ __forceinline__ int acc_row(int r, int lane) { return (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3); }

}  // namespace gemm
}  // namespace int8k
