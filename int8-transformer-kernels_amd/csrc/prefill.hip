// prefill.hip — INT8 flash attention for prefill (seq_q == seq_kv), gfx950.
//
// Contract of the reference int8_attention_forward (kernels/int8_attention.cu:
// 926-1028; math at kernels/int8_attention.cu:292-298, 467-643):
//   s_ij  = (q_i . k_j) [exact int32] * sQ_i * sK_j / sqrt(D)
//   p_ij  = softmax_j(s_ij)                          (fp32, online)
//   out_i = sum_j (p_ij * sV_j)[fp16] * v_j[fp16] / sum_j p_ij   -> fp16
// Non-causal by default (the reference has no mask); `causal` adds the
// standard lower-triangular mask (key j visible to query i iff j <= i).
//
// Design (CDNA4): a block owns the queries of one (b,h), 32 per wave (256
// queries on 8 waves at head_dim 128, 128 queries on 4 waves at 64 and 256),
// and walks the KV sequence in tiles of 64 keys.  K (int8 rows), V (fp16,
// row-major) and both key-scale vectors of a tile are staged in double-buffered LDS
// by buffer loads: the next tile's loads are in flight in registers while the
// current tile is computed, and there is one barrier per tile.  The LDS reads
// of the MFMA fragments and key scales are scheduled ahead of their uses.  The
// wave index is read into a scalar register, so every per-wave condition of the
// tile loop (causal skip, masked tile, fast or slow path) is a scalar branch.
// Everything is computed transposed so that each lane owns one query:
//   S^T[64 keys x 32 q] = K . Q^T   on v_mfma_i32_32x32x32_i8 (A = K rows
//                                   from LDS, B = Q kept in VGPRs)
//   O^T[D x 32 q]      += V^T . P^T on v_mfma_f32_32x32x16_f16
// In the 32x32 accumulator layout lane l holds column l%32 — its query — and
// 16 of the 32 keys, so the row max, the exponentials, the running sum and the
// rescale of O are lane-local except for one exchange with lane l^32, which
// holds the other 16 keys of the same query.  P^T feeds the PV MFMA from the
// registers it was computed in; V is staged once per tile into LDS as fp16
// [key][dim] rows, as it arrives, and each V^T fragment is two transposing LDS
// reads (ds_read_b64_tr_b16) whose key order matches those P^T registers.
//
// Head dims: 64, 128 and 256 run the kernel at their own size; any other
// multiple of 16 up to 256 runs the next of those sizes with the missing dims
// read as zero (Q, V) and never stored.  Any other head_dim up to 512 (the
// reference's scalar fallback, kernels/int8_attention.cu:65-157) runs
// prefill_generic_kernel.
//
// With an int8 destination the epilogue emits the per-token quantization of
// the fp16 output row instead (the attention output as the next INT8 stage's
// input): the fp16 values the fp16 path would store, their row absmax, and
// the per-token quantizer's codes and scale — the same bytes as
// int8k_quantize_per_token over the fp16 output, without its round trip.
#include <cmath>

#include "int8k_common.h"
#include "rows.h"

namespace int8k {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kKV = 64;  // keys per tile
// Block shape per head_dim: one wave per 32 queries.  D = 128 runs 8 waves
// (256 queries) at 2 waves per SIMD, so each staged K/V tile serves 256
// queries; D = 64 keeps 4 waves (a 64-key tile has only 256 K chunks of 16 B)
// and D = 256 keeps 4 waves at one wave per SIMD for its register budget.
template <int D>
struct Shape {
    static constexpr int kWaves = D == 128 ? 8 : 4;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kQ = 32 * kWaves;  // queries per block
    static constexpr int kMinBlocks = D == 64 ? 2 : 1;  // 2 waves per SIMD at D <= 128
};
// The V scales are applied once per staged tile, V' = fp16(v * sV * 2^-E), and
// the probabilities enter the PV MFMA as P = fp16(p * 2^E), so
// P . V' = sum_j p_j v_j sV_j as the reference's fp16(p * sV) . fp16(v)
// (kernels/int8_attention.cu:530-572).  E >= 0 is chosen per block, from
// max|sV| over the keys that block reads ([0, kv_end)), so that
// 127 * max|sV| * 2^-E <= 32768 (0 for V from fp16 data) and V' is finite
// wherever the reference's P' is; E <= kMaxVExp.  Causal query tiles of one
// (b,h) may use different E: each normalises with its own 2^E.
constexpr int kMaxVExp = 11;

// V' is staged as it arrives, row-major fp16 [key][dim], and the PV MFMA's
// V^T fragments are formed by transposing LDS reads (ds_read_b64_tr_b16).
// Measured on the box: in each group of 16 lanes, the instruction gives lane
// 4h + e half e of the 8-byte rows that lanes h, h+4, h+8, h+12 address.  So
// lane 16G + 4k + h of a wave addresses key row 4 (G/2) + k and dims
// 16 (G%2) + 4h of a 16-key slice, and lane l then holds dim l % 32 of keys
// 4 (l/32) + 0..3: the first half of its fragment; a read 8 rows further
// gives the second (see tile_pv).  Rows hold D + 32 halfs (2D + 64 bytes, 64
// or 192 mod 256), so the 4 rows a half-wave reads fall in 4 different 64-byte
// bank groups.
//
// Work item n of thread t is the 4x4 block of keys 4 kg .. 4 kg + 3 and dims
// 4 dg .. 4 dg + 3 with kg = t / W, dg = t % W + n W, where W = D / 4 / items
// per thread (32 at D = 128, 16 at D = 64 and 256): dim groups run fastest, so
// a wave's loads of one key cover whole 64- or 128-byte runs of rows in memory
// and its LDS writes whole runs of staged rows, and a thread's items share
// their keys (one sV vector).
template <int D>
struct VLayout {
    static constexpr int kRow = D + 32;  // halfs per staged row
    static constexpr int kItems = 64 * D / 16 / Shape<D>::kThreads;
    static constexpr int kW = D / 4 / kItems;  // dim groups per item row
};

// One LDS stage: K tile (int8 rows, 16-byte padded), V' tile (fp16 [key][dim],
// the V scales applied), the key scales sK.
template <int D>
struct Stage {
    static constexpr int kKStride = D + 16;  // bytes per K row
    static constexpr int kKBytes = kKV * kKStride;
    static constexpr int kVtBytes = kKV * VLayout<D>::kRow * 2;
    static constexpr int kBytes = kKBytes + kVtBytes + kKV * 4;
    static constexpr int kKChunks = kKV * D / 16 / Shape<D>::kThreads;  // 16-B K chunks per thread
    static constexpr int kVItems = kKV * D / 16 / Shape<D>::kThreads;   // 4x4 V blocks per thread
    static_assert(kKChunks >= 1 && kKChunks * 16 * Shape<D>::kThreads == kKV * D, "K tile split");
    static_assert(kVItems >= 1 && kVItems * 16 * Shape<D>::kThreads == kKV * D, "V tile split");
};

// Buffer resources over one (b,h)'s K, V and scales.  Rows at or past S read
// as zero, so the tile loads need no clamping; masked keys never reach the
// output.  `dm` is the head_dim of the rows in memory; a padded kernel
// (dm < D) loads only the K chunks and V dim groups below dm and zeroes the
// rest (kvalid, vvalid).
struct TileSrc {
    __amdgpu_buffer_rsrc_t k, s, sv;
    v4i v;  // V descriptor with a typed format: 8_8_8_8 SSCALED (see load_v_f16x4)
    uint32_t voff_k, voff_v, voff_s, voff_sv;
    uint32_t kstep, dm;  // bytes between K chunks n and n+1; row stride in memory
    bool kvalid;
    uint32_t vvalid;  // bit n: item n has dims below dm
};

// A buffer descriptor whose loads convert: data format 8_8_8_8 with numeric
// format SSCALED turns each byte into the float of its signed value, and the
// d16 variant of the format load packs the four as fp16.  So V arrives as exact
// fp16 with no VALU work.  Offsets at or past `bytes` read as zero.
__device__ __forceinline__ v4i make_v_descriptor(const void* base, uint32_t bytes) {
    constexpr uint32_t kDstSelXYZW = 4 | (5 << 3) | (6 << 6) | (7 << 9);
    constexpr uint32_t kNumFormatSscaled = 3, kDataFormat8888 = 10;
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    v4i d;
    d.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b));
    d.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32) & 0xffffu);  // stride 0
    d.z = __builtin_amdgcn_readfirstlane(bytes);
    d.w = kDstSelXYZW | (kNumFormatSscaled << 12) | (kDataFormat8888 << 15);
    return d;
}

// The LLVM intrinsic behind the typed ("format") raw buffer load, which clang
// exposes no builtin for; declared by name so the compiler schedules it and
// tracks its wait counts like any other load.
typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
extern "C" __device__ v4h_t int8k_raw_buffer_load_format_v4f16(v4i rsrc, int voffset, int soffset,
                                                              int aux)
    __asm("llvm.amdgcn.raw.buffer.load.format.v4f16");

// Four int8 at voff + soff as four fp16, packed {b0, b1} {b2, b3}.
__device__ __forceinline__ uint2 load_v_f16x4(const v4i& desc, uint32_t voff, uint32_t soff) {
    const v4h_t h = int8k_raw_buffer_load_format_v4f16(desc, (int)voff, (int)soff, 0);
    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    const v2u r = __builtin_bit_cast(v2u, h);
    return make_uint2(r.x, r.y);
}

template <int D>
__device__ __forceinline__ TileSrc make_tile_src(const int8_t* Kbh, const int8_t* Vbh,
                                                 const float* sKbh, const float* sVbh, int S,
                                                 int dm) {
    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    constexpr int kT = Shape<D>::kThreads;
    TileSrc src;
    src.dm = (uint32_t)dm;
    src.k = make_buffer(Kbh, (uint32_t)S * dm);
    src.v = make_v_descriptor(Vbh, (uint32_t)S * dm);
    (void)wave;
    src.s = make_buffer(sKbh, (uint32_t)S * 4);    // wave 0 loads the tile's sK
    src.sv = make_buffer(sVbh, (uint32_t)S * 4);   // every thread: sV of its 4 V keys
    const int kcol = (t % (D / 16)) * 16;
    src.voff_k = (t / (D / 16)) * dm + kcol;
    src.kstep = (uint32_t)(kT * 16 / D) * dm;  // chunk t + n kT is kT*16/D rows further
    src.kvalid = kcol < dm;
    using VL = VLayout<D>;
    const int dg = t % VL::kW, kg = t / VL::kW;
    src.voff_v = 4 * kg * dm + 4 * dg;
    src.vvalid = 0;
#pragma unroll
    for (int n = 0; n < VL::kItems; ++n)
        if (4 * (dg + n * VL::kW) < dm) src.vvalid |= 1u << n;
    src.voff_s = (t & (kKV - 1)) * 4;
    src.voff_sv = 16 * kg;
    return src;
}

// Registers holding the next tile while the current one is computed.
template <int D>
struct Prefetch {
    int4 k[Stage<D>::kKChunks];
    uint2 v[Stage<D>::kVItems][4];  // key 4 kg + i, dims 4 dg .. 4 dg + 3 as fp16 pairs
    float4 sv;  // sV of keys 4 kg .. 4 kg + 3 (the keys of every item of the thread)
    float sc;   // threads 0..63: sK of key tid
};

// Thread t (of kT) loads 16-byte K chunk t + kT n (row (t + kT n) / (D/16);
// chunks of consecutive n are kT*16/D rows apart), the 4x4 int8 V blocks of its
// items (rows 4 kg .. 4 kg + 3, dims 4 dg .. 4 dg + 3; items n and n+1 are
// 4 VLayout::kW bytes apart) and their 4 sV.  PAD: chunks and blocks past the
// memory head_dim are zero.
template <int D, bool PAD>
__device__ __forceinline__ void prefetch_tile(Prefetch<D>& pf, const TileSrc& src, int k0) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    typedef float v4f __attribute__((ext_vector_type(4)));
    constexpr int kT = Shape<D>::kThreads;
    const uint32_t dm = PAD ? src.dm : (uint32_t)D;
#pragma unroll
    for (int n = 0; n < Stage<D>::kKChunks; ++n) {
        if (!PAD || src.kvalid) {
            const v4u w = __builtin_amdgcn_raw_buffer_load_b128(
                src.k, src.voff_k, k0 * dm + n * (PAD ? src.kstep : (uint32_t)(kT * 16)), 0);
            pf.k[n] = make_int4((int)w.x, (int)w.y, (int)w.z, (int)w.w);
        } else {
            pf.k[n] = make_int4(0, 0, 0, 0);
        }
    }
#pragma unroll
    for (int n = 0; n < Stage<D>::kVItems; ++n) {
        if (!PAD || (src.vvalid >> n) & 1u) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                pf.v[n][i] = load_v_f16x4(src.v, src.voff_v,
                                          (k0 + i) * dm + n * 4 * VLayout<D>::kW);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) pf.v[n][i] = make_uint2(0, 0);
        }
    }
    const v4f sv = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(src.sv, src.voff_sv,
                                                                                k0 * 4, 0));
    pf.sv = make_float4(sv.x, sv.y, sv.z, sv.w);
    if (threadIdx.x < kKV)
        pf.sc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(src.s, src.voff_s,
                                                                               k0 * 4, 0));
}

// vscale = 2^-E: V' = fp16(v * fp16(sV * 2^-E)) on v_pk_mul_f16, written as it
// arrived: each key's 4 dims of an item as one 8-byte row piece.
template <int D>
__device__ __forceinline__ void commit_tile(const Prefetch<D>& pf, char* st, float vscale) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    using VL = VLayout<D>;
    const int t = threadIdx.x;
#pragma unroll
    for (int n = 0; n < Stage<D>::kKChunks; ++n) {
        const int c = t + n * Shape<D>::kThreads;
        const int row = c / (D / 16), col = (c % (D / 16)) * 16;
        *reinterpret_cast<int4*>(st + row * Stage<D>::kKStride + col) = pf.k[n];
    }
    _Float16* vs = reinterpret_cast<_Float16*>(st + Stage<D>::kKBytes) +
                   (t / VL::kW) * 4 * VL::kRow + (t % VL::kW) * 4;
    // key 4 kg + i scaled by its sV * 2^-E (both dims of a word share the key)
    const float svk[4] = {pf.sv.x * vscale, pf.sv.y * vscale, pf.sv.z * vscale,
                          pf.sv.w * vscale};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const h2 sp = __builtin_convertvector((float __attribute__((ext_vector_type(2)))){svk[i], svk[i]}, h2);
#pragma unroll
        for (int n = 0; n < Stage<D>::kVItems; ++n) {
            uint2 w;
            w.x = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, pf.v[n][i].x) * sp);
            w.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, pf.v[n][i].y) * sp);
            *reinterpret_cast<uint2*>(vs + i * VL::kRow + n * 4 * VL::kW) = w;
        }
    }
    if (t < kKV) reinterpret_cast<float*>(st + Stage<D>::kKBytes + Stage<D>::kVtBytes)[t] = pf.sc;
}

// Sum of the 32 fp16 P of a lane in fp32 (v_dot2_f32_f16 against {1, 1}).
__device__ __forceinline__ float psum(const v8h (&pfr)[4]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 one = {(_Float16)1.f, (_Float16)1.f};
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a = __builtin_amdgcn_fdot2(h2{pfr[i][0], pfr[i][1]}, one, a, false);
        b = __builtin_amdgcn_fdot2(h2{pfr[i][2], pfr[i][3]}, one, b, false);
        a = __builtin_amdgcn_fdot2(h2{pfr[i][4], pfr[i][5]}, one, a, false);
        b = __builtin_amdgcn_fdot2(h2{pfr[i][6], pfr[i][7]}, one, b, false);
    }
    return a + b;
}

// D: the kernel's head_dim.  PAD: the rows in memory have head_dim d_mem < D
// (a multiple of 16); the dims past it read as zero and are not stored.
template <int D, bool CAUSAL, bool PAD>
__global__ __launch_bounds__(Shape<D>::kThreads, Shape<D>::kMinBlocks) void prefill_kernel(
    const int8_t* __restrict__ Q, const int8_t* __restrict__ K, const int8_t* __restrict__ V,
    const float* __restrict__ sQ, const float* __restrict__ sK, const float* __restrict__ sV,
    uint16_t* __restrict__ out, int8_t* __restrict__ qout, float* __restrict__ qout_scale, int S,
    int n_qtiles, float qk_scale_log2, int heads, int bshd, int d_mem) {
    constexpr int NS = D / 32;  // 32-wide d slices (QK k-steps) and O^T row tiles
    const int dm = PAD ? d_mem : D;  // head_dim of the rows in memory
    using St = Stage<D>;
    extern __shared__ __align__(16) char smem[];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;
    // Under the causal mask a query tile's work grows with its index, so the
    // grid is query-tile-major, heaviest tiles of every (b,h) first.  Without
    // it, the query tiles of one (b,h) share its K/V, so they run on one XCD
    // (one L2): blocks are dispatched to the 8 XCDs in turn, and XCD x takes a
    // contiguous range of (b,h, query tile) pairs in (b,h)-major order.
    const int BH = gridDim.x / n_qtiles;
    int bh, qt;
    if constexpr (CAUSAL) {
        bh = (int)(blockIdx.x % BH);
        qt = n_qtiles - 1 - (int)(blockIdx.x / BH);
    } else {
        constexpr int kXcds = 8;
        const int xcd = (int)(blockIdx.x % kXcds), local = (int)(blockIdx.x / kXcds);
        const int per = (int)(gridDim.x / kXcds), rem = (int)(gridDim.x % kXcds);
        const int tile = xcd * per + min(xcd, rem) + local;
        bh = tile / n_qtiles;
        qt = tile - bh * n_qtiles;
    }
    constexpr int kQ = Shape<D>::kQ;
    const int qw0 = qt * kQ + wave * 32;  // first query of this wave
    const int q = qw0 + (lane & 31);      // this lane's query
    const bool qok = q < S;

    const size_t base = (size_t)bh * S;
    const int8_t* Qbh = Q + base * dm;
    const int8_t* Kbh = K + base * dm;
    const int8_t* Vbh = V + base * dm;
    const float* sKbh = sK + base;
    const float* sVbh = sV + base;

    // Q^T fragments (B operand of the QK MFMA): column q, 16 bytes of d-slice s.
    v4i qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s)
        qf[s] = (!PAD || 32 * s + 16 * h < dm)
                    ? *reinterpret_cast<const v4i*>(Qbh + (size_t)min(q, S - 1) * dm + 32 * s + 16 * h)
                    : v4i{0, 0, 0, 0};
    // The query scale is loaded here but first used after the V-scale exponent's
    // reduction, so its wait joins the first tile's instead of adding a latency.
    const float sq_raw = qok ? sQ[base + q] : 0.f;

    v16f o[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
    float m = -INFINITY, lsum = 0.f;

    const int q_block_end = min(S, (qt + 1) * kQ);
    const int kv_end = CAUSAL ? q_block_end : S;
    const int n_kv = (kv_end + kKV - 1) / kKV;
    const int q_wave_last = min(qw0 + 31, S - 1);
    // Step i of the KV walk computes tile tile_of(i).  Causal blocks take their
    // diagonal tiles first (tiles kd .. n_kv-1, the ones some query of the block
    // does not see whole, which take the slow path anyway), so the running max is
    // set when the unmasked tiles 0 .. kd-1 follow on the fast path; otherwise the
    // first of those would take the slow path only to set it.
    const int kd = CAUSAL ? (qt * kQ) / kKV : 0;
    const int nd = n_kv - kd;
    auto tile_of = [&](int i) { return CAUSAL ? (i < nd ? kd + i : i - nd) : i; };

    // The first tile's loads go out before the exponent's reduction, so their
    // latency overlaps it.
    const TileSrc src = make_tile_src<D>(Kbh, Vbh, sKbh, sVbh, S, dm);
    Prefetch<D> pa;
    prefetch_tile<D, PAD>(pa, src, tile_of(0) * kKV);

    // E: the exponent that keeps the scaled V^T in fp16 range, from max |sV| over
    // the keys this block reads (a block-wide reduction through LDS).  Each thread
    // reads 16-byte vectors, kSvU of them in flight per round; dwords past kv_end
    // read as zero (the buffer range is checked per dword).
    __shared__ float s_svmax[Shape<D>::kWaves];
    {
        typedef float v4f __attribute__((ext_vector_type(4)));
        constexpr int kT = Shape<D>::kThreads, kSvU = 4;
        const __amdgpu_buffer_rsrc_t svr = make_buffer(sVbh, (uint32_t)kv_end * 4);
        float a = 0.f;
        for (int j0 = 0; j0 < kv_end; j0 += 4 * kT * kSvU) {
            v4f v[kSvU];
#pragma unroll
            for (int u = 0; u < kSvU; ++u)
                v[u] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                                   svr, 4 * (j0 + 4 * (u * kT + (int)threadIdx.x)), 0, 0));
#pragma unroll
            for (int u = 0; u < kSvU; ++u)
                a = fmaxf(a, fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)),
                                   fmaxf(fabsf(v[u].z), fabsf(v[u].w))));
        }
        // max over the wave on the VALU: DPP inside each 16-lane row, then the
        // row and half swaps (no LDS round trips)
        auto dmax = [](float x, int y) { return fmaxf(x, __int_as_float(y)); };
        a = dmax(a, dpp_xor1(__float_as_int(a)));
        a = dmax(a, dpp_xor2(__float_as_int(a)));
        a = dmax(a, dpp_half_mirror(__float_as_int(a)));
        a = dmax(a, dpp_row_mirror(__float_as_int(a)));
        {
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(a), __float_as_int(a),
                                                            false, false);
            a = fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
        }
        a = max_xor32(a);
        if (lane == 0) s_svmax[wave] = a;
    }
    __syncthreads();
    float svmax = s_svmax[0];
#pragma unroll
    for (int w = 1; w < Shape<D>::kWaves; ++w) svmax = fmaxf(svmax, s_svmax[w]);
    int vexp = 0;  // smallest E (up to kMaxVExp) with 127 max|sV| 2^-E <= 32768
    {
        const float need = svmax * (127.f / 32768.f);
        if (!(need <= 1.f)) {
            int e = kMaxVExp;
            if (need < INFINITY) frexpf(need, &e);  // need < 2^e
            vexp = min(e, kMaxVExp);
        }
    }
    const float vscale = __builtin_ldexpf(1.f, -vexp);  // V^T = fp16(v * sV * 2^-E)
    const float pexp = (float)vexp;                      // P = fp16(p * 2^E)
    const float qscale = sq_raw * qk_scale_log2;
    const bool qpos = __ballot(!(qscale >= 0.f)) == 0;  // wave-uniform

    auto stage_of = [&](int kt) { return smem + (kt & 1) * St::kBytes; };
    // S^T = K . Q^T for the two 32-key halves of tile kt
    auto qk = [&](int kt, v16i (&sacc)[2]) {
        const char* st = stage_of(kt);
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            v4i kf[NS];
            const char* krow = st + (32 * T + (lane & 31)) * St::kKStride + 16 * h;
#pragma unroll
            for (int s = 0; s < NS; ++s) kf[s] = *reinterpret_cast<const v4i*>(krow + 32 * s);
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[T][r] = 0;
#pragma unroll
            for (int s = 0; s < NS; ++s)
                sacc[T] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[s], qf[s], sacc[T], 0, 0, 0);
        }
    };
    // O^T += V^T . P^T; the V^T fragment of dim slice t and 16-key slice ks is two
    // transposing reads of the row-major V' (VLayout): keys 16 ks + 4 (lane/32) + 0..3,
    // then 8 keys further, at dim 32 t + lane % 32
    typedef _Float16 v4h __attribute__((ext_vector_type(4)));
    typedef short v4s __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s lds_v4s;
    constexpr int kVRowB = 2 * VLayout<D>::kRow;  // bytes per staged V' row
    const int v_lane = (4 * (lane >> 5) + ((lane & 15) >> 2)) * kVRowB +
                       2 * (16 * ((lane >> 4) & 1) + 4 * (lane & 3));
    auto pv = [&](int kt, const v8h (&pfr)[4]) {
        const char* vs = stage_of(kt) + St::kKBytes + v_lane;
#pragma unroll
        for (int t = 0; t < NS; ++t) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const char* p = vs + 16 * ks * kVRowB + 64 * t;
                const v4h lo = __builtin_bit_cast(
                    v4h, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p));
                const v4h hi = __builtin_bit_cast(
                    v4h, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p + 8 * kVRowB)));
                const v8h vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pfr[ks], o[t], 0, 0, 0);
            }
        }
    };
    auto sk_of = [&](int kt) {
        return reinterpret_cast<const float*>(stage_of(kt) + St::kKBytes + St::kVtBytes);
    };
    // A wave computes tile k unless the causal mask hides all of it from the wave's queries.
    auto computes = [&](int k) { return !(CAUSAL && k * kKV > q_wave_last); };
    // Keep the K-fragment and sK reads of the fast tile ahead of their uses
    // (the compiler otherwise waits on each LDS read right before its MFMA).
    auto schedule_qk = [&]() {
#pragma unroll
        for (int i = 0; i < NS; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    };
    // V^T fragments (two reads each) 4 MFMAs ahead of their use
    auto schedule_pv = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 0; i < 4 * NS - 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };

    // Scores of this lane's 32 keys: key = k0 + 32T + 8g + 4h + c <-> sacc[T][4g + c];
    // P^T = fp16(p * 2^E): slice t = registers [8(t%2), 8(t%2)+8) of half t/2.
    //
    // The running max m is a reference, not necessarily the exact running max.  A
    // tile takes the fast path when it has no masked key and every lane's qscale is
    // >= 0: p = 2^(u*qscale - m + E) with the current m, no per-score max and no
    // rescale of O; the tile is kept if each lane's sum of its 32 P stays below the
    // fp16 maximum, so every P is finite.  p may exceed 1 when the scores have grown
    // since m was set; O and l hold such values in fp32.  Every other tile (the
    // wave's first, masked edge and diagonal tiles, a sum past the fp16 range) takes
    // the slow path, which sets m to the exact running max and rescales O and l.  l
    // sums the fp16 P that enter the PV product.
    //
    // Step kt is computed from LDS stage kt&1.  The register set holds step
    // kt+1's tile while step kt is computed; at the end of the step it is written
    // to the other stage, refilled with step kt+2's tile, and the step's one
    // barrier follows.  The fast path runs as an inner loop that the slow path
    // leaves and re-enters, so O has no conditional update inside it.
    commit_tile<D>(pa, smem, vscale);
    if (n_kv > 1) prefetch_tile<D, PAD>(pa, src, tile_of(1) * kKV);
    __syncthreads();
    auto advance = [&](int kt) {
        if (kt + 1 < n_kv) {
            commit_tile<D>(pa, smem + ((kt + 1) & 1) * St::kBytes, vscale);
            if (kt + 2 < n_kv) prefetch_tile<D, PAD>(pa, src, tile_of(kt + 2) * kKV);
        }
        // step kt+1's tile is in LDS and every wave is done reading stage kt&1
        __syncthreads();
    };
    bool have_m = false;  // wave-uniform: a slow step has set the running max
    int kt = 0;
    while (kt < n_kv) {
        v16i sacc[2];
        bool slow = false;
        for (; kt < n_kv; ++kt) {
            const int tk = tile_of(kt);
            if (computes(tk)) {
                const int k0 = tk * kKV;
                const bool full = k0 + kKV <= S && !(CAUSAL && k0 + kKV - 1 > qw0);
                if (!(full && qpos && have_m)) {
                    qk(kt, sacc);
                    slow = true;
                    break;
                }
                qk(kt, sacc);
                const float* sk_l = sk_of(kt);
                const float shift = pexp - m;
                v8h pfr[4];
#pragma unroll
                for (int T = 0; T < 2; ++T)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const float4 skv = *reinterpret_cast<const float4*>(sk_l + 32 * T + 8 * g + 4 * h);
                        const float skk[4] = {skv.x, skv.y, skv.z, skv.w};
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const float u = static_cast<float>(sacc[T][4 * g + c]) * skk[c];
                            pfr[2 * T + (g >> 1)][4 * (g & 1) + c] =
                                (_Float16)fast_exp2(fmaf(u, qscale, shift));
                        }
                    }
                schedule_qk();
                const float tsum = psum(pfr);
                if (__ballot(!(tsum <= 65504.f))) { slow = true; break; }
                lsum += tsum;
                pv(kt, pfr);
                schedule_pv();
            }
            advance(kt);
        }
        if (!slow) break;
        // Slow path for step kt (its S^T is in sacc): s = acc * qscale * sK with masked
        // keys at -inf, exact running max, rescale of O and l.
        {
            const int k0 = tile_of(kt) * kKV;
            const float* sk_l = sk_of(kt);
            float sc[2][16];
            float mx = -INFINITY;
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const float4 skv = *reinterpret_cast<const float4*>(sk_l + 32 * T + 8 * g + 4 * h);
                    const float skk[4] = {skv.x, skv.y, skv.z, skv.w};
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        float v = static_cast<float>(sacc[T][4 * g + c]) * qscale * skk[c];
                        const int key = k0 + 32 * T + 8 * g + 4 * h + c;
                        if (key >= S || (CAUSAL && key > q)) v = -INFINITY;
                        sc[T][4 * g + c] = v;
                        mx = fmaxf(mx, v);
                    }
                }
            mx = max_xor32(mx);
            const float m_new = fmaxf(m, mx);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float corr = fast_exp2(m - m_use);
            lsum *= corr;
#pragma unroll
            for (int t = 0; t < NS; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[t][r] *= corr;
            m = m_new;
            const float shift = pexp - m_use;
            v8h pfr[4];
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int g = 0; g < 4; ++g)
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        pfr[2 * T + (g >> 1)][4 * (g & 1) + c] =
                            (_Float16)fast_exp2(sc[T][4 * g + c] + shift);
            lsum += psum(pfr);
            pv(kt, pfr);
        }
        have_m = true;
        advance(kt);
        ++kt;
    }

    const float L = sum_xor32(lsum);
    if (!qok) return;  // lanes l and l^32 share q, so both leave or both stay
    // l carries the 2^E of P; O = sum p v sV does not
    float inv = 1.f / L;
    if (vexp != 0) inv *= __builtin_ldexpf(1.f, vexp);
    // output row: [B, H, S, D] order, or [B, S, H, D] (the row order of the
    // output projection's input) with bshd
    const size_t orow_index =
        bshd ? ((size_t)(bh / heads) * S + q) * heads + (size_t)(bh % heads) : base + q;
    // fp16 output values (rounded from the fp32 quotient); lane l holds
    // d = 32 t + 8 g + 4 h + c of its query, lane l^32 the other half
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] = __half2float(f16_of_f32(o[t][r] * inv));
    if (qout != nullptr) {
        float am = 0.f;
#pragma unroll
        for (int t = 0; t < NS; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r) am = fmaxf(am, fabsf(o[t][r]));
        am = max_xor32(am);
        const float sc = fmaxf(am, 1e-8f) / 127.f;
        const float rinv = 1.f / sc;
        int8_t* qrow = qout + orow_index * dm;
#pragma unroll
        for (int t = 0; t < NS; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * t + 8 * g + 4 * h;
                const float y[4] = {o[t][4 * g], o[t][4 * g + 1], o[t][4 * g + 2], o[t][4 * g + 3]};
                if (!PAD || d < dm) store_codes<4>(y, sc, rinv, qrow + d);
            }
        if (h == 0) qout_scale[orow_index] = sc;
        return;
    }
    uint16_t* orow = out + orow_index * dm;
#pragma unroll
    for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * t + 8 * g + 4 * h;
            if (PAD && d >= dm) continue;
            const uint32_t lo = f32_to_f16_bits(o[t][4 * g]) |
                                ((uint32_t)f32_to_f16_bits(o[t][4 * g + 1]) << 16);
            const uint32_t hi = f32_to_f16_bits(o[t][4 * g + 2]) |
                                ((uint32_t)f32_to_f16_bits(o[t][4 * g + 3]) << 16);
            *reinterpret_cast<uint2*>(orow + d) = make_uint2(lo, hi);
        }
}

// ---------------------------------------------------------------- any head_dim
// Head dims the MFMA kernel does not take (not a multiple of 16, or above 256)
// up to kGenMaxD, the reference's scalar fallback (kernels/int8_attention.cu:
// 65-157, 1019-1027) with the same math.  A block holds kGenQ queries of one
// (b,h), kGenQW per wave, and stages each 64-key tile in LDS: K as zero-padded
// 4-byte words, V as bytes, the key scales as fp32.  Lane j scores key j of
// the tile for the wave's queries (v_dot4 over the words: exact int32), the
// online softmax is a wave reduction, and each lane then accumulates dims
// d = lane + 64 e over the tile's keys with the weights p_j * sV_j broadcast by
// v_readlane.  Outputs as prefill_kernel: fp16 rounded from the fp32 quotient,
// or its per-token int8 codes and scale; [B,H,S,D] or [B,S,H,D] rows.
constexpr int kGenMaxD = 512;
constexpr int kGenQW = 4;                // queries per wave
constexpr int kGenQ = 4 * kGenQW;        // queries per block (4 waves)
constexpr int kGenKV = 64;               // keys per tile
constexpr int kGenDims = kGenMaxD / 64;  // dims per lane, at most

// LDS layout of prefill_generic_kernel for head_dim D (bytes).
struct GenLayout {
    int dw, ks;  // 4-byte words per row (zero-padded), K row stride in words (odd)
    int v_off, s_off, q_off, bytes;
};
__host__ __device__ inline GenLayout gen_layout(int D) {
    GenLayout g;
    g.dw = (D + 3) / 4;
    g.ks = g.dw | 1;  // odd: the 64 lanes' rows start in 64 different banks
    g.v_off = kGenKV * g.ks * 4;
    g.s_off = g.v_off + (kGenKV * D + 15) / 16 * 16;
    g.q_off = g.s_off + 2 * kGenKV * 4;
    g.bytes = g.q_off + kGenQ * g.dw * 4;
    return g;
}

template <bool CAUSAL>
__global__ __launch_bounds__(256) void prefill_generic_kernel(
    const int8_t* __restrict__ Q, const int8_t* __restrict__ K, const int8_t* __restrict__ V,
    const float* __restrict__ sQ, const float* __restrict__ sK, const float* __restrict__ sV,
    uint16_t* __restrict__ out, int8_t* __restrict__ qout, float* __restrict__ qout_scale, int S,
    int D, int n_qtiles, float qk_scale_log2, int heads, int bshd) {
    extern __shared__ __align__(16) char smem[];
    const GenLayout L = gen_layout(D);
    int* kw = reinterpret_cast<int*>(smem);
    int8_t* vb = reinterpret_cast<int8_t*>(smem + L.v_off);
    float* ssk = reinterpret_cast<float*>(smem + L.s_off);
    float* ssv = ssk + kGenKV;
    int* qw = reinterpret_cast<int*>(smem + L.q_off);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // causal grids: heaviest query tiles of every (b,h) first
    const int BH = gridDim.x / n_qtiles;
    int bh, qt;
    if constexpr (CAUSAL) {
        bh = (int)(blockIdx.x % BH);
        qt = n_qtiles - 1 - (int)(blockIdx.x / BH);
    } else {
        bh = (int)(blockIdx.x / n_qtiles);
        qt = (int)(blockIdx.x % n_qtiles);
    }
    const int q0 = qt * kGenQ;
    const size_t base = (size_t)bh * S;
    const int rowb = L.dw * 4;  // bytes per zero-padded row

    int8_t* qb = reinterpret_cast<int8_t*>(qw);
    for (int i = t; i < kGenQ * rowb; i += 256) {
        const int r = i / rowb, c = i - r * rowb;
        qb[i] = (q0 + r < S && c < D) ? Q[(base + q0 + r) * D + c] : (int8_t)0;
    }
    float qs[kGenQW], m[kGenQW], l[kGenQW], acc[kGenQW][kGenDims];
#pragma unroll
    for (int i = 0; i < kGenQW; ++i) {
        const int q = q0 + wave * kGenQW + i;
        qs[i] = q < S ? sQ[base + q] * qk_scale_log2 : 0.f;
        m[i] = -INFINITY;
        l[i] = 0.f;
#pragma unroll
        for (int e = 0; e < kGenDims; ++e) acc[i][e] = 0.f;
    }
    const int nd = (D + 63) >> 6;
    const int kv_end = CAUSAL ? min(S, q0 + kGenQ) : S;
    for (int k0 = 0; k0 < kv_end; k0 += kGenKV) {
        __syncthreads();  // the previous tile's reads are done
        int8_t* kb = reinterpret_cast<int8_t*>(kw);
        const int krow = L.ks * 4;
        for (int i = t; i < kGenKV * krow; i += 256) {
            const int r = i / krow, c = i - r * krow;
            kb[i] = (k0 + r < S && c < D) ? K[(base + k0 + r) * D + c] : (int8_t)0;
        }
        const int vn = min(kGenKV, S - k0) * D;
        for (int i = t; i < kGenKV * D; i += 256) vb[i] = i < vn ? V[(base + k0) * D + i] : (int8_t)0;
        if (t < kGenKV) ssk[t] = k0 + t < S ? sK[base + k0 + t] : 0.f;
        else if (t < 2 * kGenKV) ssv[t - kGenKV] = k0 + t - kGenKV < S ? sV[base + k0 + t - kGenKV] : 0.f;
        __syncthreads();

        const int key = k0 + lane;
        const float skl = ssk[lane], svl = ssv[lane];
        const int* kr = kw + lane * L.ks;
        float w[kGenQW];
#pragma unroll
        for (int i = 0; i < kGenQW; ++i) {
            const int qi = wave * kGenQW + i, q = q0 + qi;
            const int* qr = qw + qi * L.dw;
            int dot = 0;
            for (int c = 0; c < L.dw; ++c) dot = __builtin_amdgcn_sdot4(qr[c], kr[c], dot, false);
            float s = static_cast<float>(dot) * qs[i] * skl;
            if (key >= S || (CAUSAL && key > q)) s = -INFINITY;
            float mx = s;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            const float m_new = fmaxf(m[i], mx);
            const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
            const float corr = fast_exp2(m[i] - m_use);
            const float p = fast_exp2(s - m_use);
            float ps = p;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) ps += __shfl_xor(ps, off);
            l[i] = l[i] * corr + ps;
#pragma unroll
            for (int e = 0; e < kGenDims; ++e) acc[i][e] *= corr;
            m[i] = m_new;
            w[i] = p * svl;
        }
        const int nk = min(kGenKV, kv_end - k0);
        for (int j = 0; j < nk; ++j) {
            float v[kGenDims];
#pragma unroll
            for (int e = 0; e < kGenDims; ++e) {
                const int d = lane + 64 * e;
                v[e] = (e < nd && d < D) ? static_cast<float>(vb[j * D + d]) : 0.f;
            }
#pragma unroll
            for (int i = 0; i < kGenQW; ++i) {
                const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[i]), j));
#pragma unroll
                for (int e = 0; e < kGenDims; ++e) acc[i][e] = fmaf(wj, v[e], acc[i][e]);
            }
        }
    }

#pragma unroll
    for (int i = 0; i < kGenQW; ++i) {
        const int q = q0 + wave * kGenQW + i;
        if (q >= S) break;  // wave-uniform
        const float inv = 1.f / l[i];
        const size_t orow =
            bshd ? ((size_t)(bh / heads) * S + q) * heads + (size_t)(bh % heads) : base + q;
        float y[kGenDims];
#pragma unroll
        for (int e = 0; e < kGenDims; ++e) y[e] = __half2float(f16_of_f32(acc[i][e] * inv));
        if (qout != nullptr) {
            float am = 0.f;
#pragma unroll
            for (int e = 0; e < kGenDims; ++e)
                if (e < nd && lane + 64 * e < D) am = fmaxf(am, fabsf(y[e]));
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) am = fmaxf(am, __shfl_xor(am, off));
            const float sc = fmaxf(am, 1e-8f) / 127.f;
#pragma unroll
            for (int e = 0; e < kGenDims; ++e) {
                const int d = lane + 64 * e;
                if (e < nd && d < D) qout[orow * D + d] = (int8_t)quant_code(y[e], sc);
            }
            if (lane == 0) qout_scale[orow] = sc;
        } else {
#pragma unroll
            for (int e = 0; e < kGenDims; ++e) {
                const int d = lane + 64 * e;
                if (e < nd && d < D) out[orow * D + d] = f32_to_f16_bits(y[e]);
            }
        }
    }
}

// Dynamic LDS above 64 KiB needs the attribute, once per device and kernel.
template <typename... Kernels>
int set_lds_limit(PerDeviceOnce& once, int bytes, Kernels... kernels) {
    return once.run([=] {
        hipError_t e = hipSuccess;
        for (const void* k : {reinterpret_cast<const void*>(kernels)...}) {
            if (e == hipSuccess)
                e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
        }
        if (e != hipSuccess) {
            set_last_error("hipFuncSetAttribute", e);
            return (int)INT8K_ERR_HIP;
        }
        return (int)INT8K_OK;
    });
}

// D: the kernel's head_dim; dm: the head_dim of the rows in memory (dm <= D,
// a multiple of 16; dm < D runs the padded instance).
template <int D>
int launch_prefill(const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out,
                   int8_t* qout, float* qscale, const float* sQ, const float* sK, const float* sV,
                   int BH, int heads, int S, int dm, bool causal, bool bshd, hipStream_t stream) {
    constexpr int kQ = Shape<D>::kQ, kThreads = Shape<D>::kThreads;
    const int n_qtiles = (S + kQ - 1) / kQ;
    const long long blocks = (long long)BH * n_qtiles;
    const float qk = (1.0f / std::sqrt((float)dm)) * kLog2e;
    const int lds = 2 * Stage<D>::kBytes;
    static PerDeviceOnce lds_once;
    const int st = set_lds_limit(lds_once, lds, prefill_kernel<D, true, false>,
                                 prefill_kernel<D, false, false>, prefill_kernel<D, true, true>,
                                 prefill_kernel<D, false, true>);
    if (st != INT8K_OK) return st;
    const int b = bshd ? 1 : 0;
#define INT8K_PREFILL_LAUNCH(C, P)                                                         \
    prefill_kernel<D, C, P><<<(unsigned)blocks, kThreads, lds, stream>>>(                  \
        Q, K, V, sQ, sK, sV, out, qout, qscale, S, n_qtiles, qk, heads, b, dm)
    if (dm == D) {
        if (causal) INT8K_PREFILL_LAUNCH(true, false);
        else INT8K_PREFILL_LAUNCH(false, false);
    } else {
        if (causal) INT8K_PREFILL_LAUNCH(true, true);
        else INT8K_PREFILL_LAUNCH(false, true);
    }
#undef INT8K_PREFILL_LAUNCH
    return check_launch("prefill_kernel");
}

int launch_prefill_generic(const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out,
                           int8_t* qout, float* qscale, const float* sQ, const float* sK,
                           const float* sV, int BH, int heads, int S, int D, bool causal,
                           bool bshd, hipStream_t stream) {
    const int n_qtiles = (S + kGenQ - 1) / kGenQ;
    const long long blocks = (long long)BH * n_qtiles;
    const float qk = (1.0f / std::sqrt((float)D)) * kLog2e;
    static PerDeviceOnce lds_once;
    const int st = set_lds_limit(lds_once, gen_layout(kGenMaxD).bytes,
                                 prefill_generic_kernel<true>, prefill_generic_kernel<false>);
    if (st != INT8K_OK) return st;
    const int lds = gen_layout(D).bytes;
    if (causal)
        prefill_generic_kernel<true><<<(unsigned)blocks, 256, lds, stream>>>(
            Q, K, V, sQ, sK, sV, out, qout, qscale, S, D, n_qtiles, qk, heads, bshd ? 1 : 0);
    else
        prefill_generic_kernel<false><<<(unsigned)blocks, 256, lds, stream>>>(
            Q, K, V, sQ, sK, sV, out, qout, qscale, S, D, n_qtiles, qk, heads, bshd ? 1 : 0);
    return check_launch("prefill_generic_kernel");
}

// Shared checks and dispatch of both entry points: exactly one of out
// (fp16) and qout/qscale (int8 + per-token scale) is set.
int prefill_entry(const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out, int8_t* qout,
                  float* qscale, const float* scale_Q, const float* scale_K, const float* scale_V,
                  int batch, int heads, int seq_len, int head_dim, int flags, void* stream) {
    if (!Q || !K || !V || !scale_Q || !scale_K || !scale_V) return INT8K_ERR_INVALID_ARGUMENT;
    if (flags & ~(INT8K_ATTN_CAUSAL | INT8K_ATTN_OUT_BSHD)) return INT8K_ERR_INVALID_ARGUMENT;
    if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (head_dim > kGenMaxD) return INT8K_ERR_UNSUPPORTED;
    const long long BH = (long long)batch * heads;
    const bool mfma = head_dim % 16 == 0 && head_dim <= 256;
    // work-items of the launch: 2 threads per query (MFMA kernel), 16 (generic)
    if (BH * (((long long)seq_len + 127) / 128) * 256 >= (1LL << 32)) return INT8K_ERR_UNSUPPORTED;
    if (!mfma && BH * (((long long)seq_len + kGenQ - 1) / kGenQ) * 256 >= (1LL << 32))
        return INT8K_ERR_UNSUPPORTED;
    if ((long long)seq_len * head_dim >= (1LL << 32)) return INT8K_ERR_UNSUPPORTED;  // buffer range
    if (!aligned_to(scale_Q, 4) || !aligned_to(scale_K, 4) || !aligned_to(scale_V, 4))
        return INT8K_ERR_MISALIGNED;
    if (mfma) {
        if (!aligned_to(Q, 16) || !aligned_to(K, 16) || !aligned_to(V, 16))
            return INT8K_ERR_MISALIGNED;
        if (out ? !aligned_to(out, 8) : !(aligned_to(qout, 4) && aligned_to(qscale, 4)))
            return INT8K_ERR_MISALIGNED;
    } else if (out ? !aligned_to(out, 2) : !aligned_to(qscale, 4)) {
        return INT8K_ERR_MISALIGNED;
    }
    hipStream_t s = as_stream(stream);
    const bool c = (flags & INT8K_ATTN_CAUSAL) != 0, bshd = (flags & INT8K_ATTN_OUT_BSHD) != 0;
    if (!mfma)
        return launch_prefill_generic(Q, K, V, out, qout, qscale, scale_Q, scale_K, scale_V,
                                      (int)BH, heads, seq_len, head_dim, c, bshd, s);
    if (head_dim <= 64)
        return launch_prefill<64>(Q, K, V, out, qout, qscale, scale_Q, scale_K, scale_V, (int)BH,
                                  heads, seq_len, head_dim, c, bshd, s);
    if (head_dim <= 128)
        return launch_prefill<128>(Q, K, V, out, qout, qscale, scale_Q, scale_K, scale_V,
                                   (int)BH, heads, seq_len, head_dim, c, bshd, s);
    return launch_prefill<256>(Q, K, V, out, qout, qscale, scale_Q, scale_K, scale_V, (int)BH,
                               heads, seq_len, head_dim, c, bshd, s);
}

}  // namespace
}  // namespace int8k

using namespace int8k;

extern "C" int int8k_attention_forward(const int8_t* Q, const int8_t* K, const int8_t* V,
                                       uint16_t* out, const float* scale_Q, const float* scale_K,
                                       const float* scale_V, int batch, int heads, int seq_len,
                                       int head_dim, int flags, void* stream) {
    clear_last_error();
    if (!out) return INT8K_ERR_INVALID_ARGUMENT;
    return prefill_entry(Q, K, V, out, nullptr, nullptr, scale_Q, scale_K, scale_V, batch, heads,
                         seq_len, head_dim, flags, stream);
}

extern "C" int int8k_attention_forward_quant(const int8_t* Q, const int8_t* K, const int8_t* V,
                                             int8_t* out_q, float* out_scale,
                                             const float* scale_Q, const float* scale_K,
                                             const float* scale_V, int batch, int heads,
                                             int seq_len, int head_dim, int flags,
                                             void* stream) {
    clear_last_error();
    if (!out_q || !out_scale) return INT8K_ERR_INVALID_ARGUMENT;
    return prefill_entry(Q, K, V, nullptr, out_q, out_scale, scale_Q, scale_K, scale_V, batch,
                         heads, seq_len, head_dim, flags, stream);
}
