// decode.hip — split-KV flash-decoding over a contiguous INT8 KV cache (gfx950).
//
// Computes, for every (b,h) = bh and a single query token,
//     out[bh,:] = sum_j softmax_j(score_j) * (V[bh,j,:] * sV[bh*S+j])
//     score_j   = (Q[bh,:] . K[bh,j,:]) * sQ[bh] * sK[bh*S+j] / sqrt(D)
// which is the contract of the reference launcher
// int8_decode_attention_forward (kernels/int8_decode_attention.cu:443-547) and
// of its partial/combine pair (kernels/int8_decode_attention.cu:274-426).
//
// Design (CDNA4 first, not a translation of the warp-per-unit CUDA kernel):
//
//  * HBM-bound: one pass over K and V (2*BH*S*D bytes) dominates.  Each wave64
//    lane issues 16-byte global loads; a wave's load instruction covers
//    64 x 16 B = 1 KiB made of whole 128-byte (D=128) or 64-byte (D=64) rows.
//  * Lane layout: LPR = D/16 lanes share a row (lane s of the group holds row
//    bytes [16s, 16s+16)); G = 64/LPR row-groups per wave.  One wave
//    iteration covers R = G*NSLOT rows: group g owns rows g*NSLOT .. +NSLOT-1
//    of the block, one per load slot, so every slot of every lane is an
//    immediate offset from one base address.
//  * Paired rows (D=64, 4 slots, the 8-wave one-launch kernels): a 64-byte
//    row is half a 128-byte line, so groups 2h and 2h+1 take the even and the
//    odd rows of block rows 8h..8h+7 (slot t: row 8h + o + 2t) and every load
//    instruction covers whole lines.  That makes non-temporal K/V loads pay
//    at D=64 too; with half lines per instruction they cost 20-100%.  Each
//    lane then loads one of its group's four scales and the group reads them
//    with a DPP quad broadcast.
//  * QK: 4 v_dot4_i32_i8 per slot per lane (exact int32), then a DPP sum over
//    the LPR lanes of the group (no LDS).  The group's lanes all hold the score.
//  * Softmax: every row-group keeps its own online-softmax state (m, l) in the
//    log2 domain and its own fp32 accumulator for the 16 dims its lane holds,
//    so the hot loop has no cross-group traffic at all.  The G group states of
//    a wave are merged once, at the end of the wave's KV chunk.
//  * PV: each V byte is converted with one SDWA v_cvt_f32_i32 and folded in
//    with one FMA: acc += (p_j * sV_j) * v_j.
//  * Split-KV: a work unit = one wave = one (bh, chunk).  The split count is
//    chosen on the host so that BH*nsplit waves fill 256 CUs several times
//    over; partial states (m, l, acc[D]) go to the workspace and a combine
//    kernel merges them with the log-sum-exp rule into fp16.
#include <algorithm>
#include <cmath>
#include <cstdlib>

#include "int8k_common.h"
#include "rows.h"

namespace int8k {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kNtKV = 1;      // non-temporal K/V loads (each row is read once)
constexpr int kNtScales = 2;  // non-temporal sK/sV loads
constexpr int kBlockThreads = 64 * kWavesPerBlock;

// NS = load slots: rows per row-group per wave iteration (each slot is one
// 16-byte K load and one 16-byte V load per lane).
template <int D, int NS>
struct DecodeGeom {
    static_assert(D == 64 || D == 128, "decode supports head_dim 64 and 128");
    static_assert(NS == 4 || NS == 8, "slots per iteration: 4 or 8");
    static constexpr int kLanesPerRow = D / 16;
    static constexpr int kGroups = 64 / kLanesPerRow;
    static constexpr int kRowsPerIter = kGroups * NS;
};

// Rows per wave iteration for a head dim (host side).
inline int rows_per_iter(int D, int ns) { return (64 / (D / 16)) * ns; }

// Paired rows (the 8-wave one-launch kernels at D=64 with 4 slots): group
// 2h+o owns rows 8h+o, +2, +4, +6 of a wave iteration's block, so each load
// slot covers whole 128-byte lines; otherwise group g owns rows g*NS .. +NS-1.
constexpr bool paired_rows(int D, int NS, int MAXW) { return D == 64 && NS == 4 && MAXW <= 8; }

// Two register sets (the next iteration's loads in flight) in the 8-wave
// one-launch kernels: at 4 slots, and at D = 128 with 8 slots.
constexpr bool two_sets(int D, int NS, int MAXW) { return MAXW <= 8 && (NS == 4 || D == 128); }

template <bool PAIRED, int NS>
__device__ __forceinline__ int group_row0(int grp) {
    if constexpr (PAIRED) return 8 * (grp >> 1) + (grp & 1);
    else return grp * NS;
}

// Launch-time tuning of the decode kernel.
struct DecodeTuning {
    int slots;         // NS
    int flags;         // kNtKV | kNtScales
    int target_units;  // units (waves) to aim for
    int stagger;       // rotate each unit's starting iteration
    int pair_flags;    // load flags of the paired-row kernels (D=64, 4 slots, <= 8 chunks)
};

struct SplitPlan {
    int nsplit;
    int chunk;
};

// Most chunks per (b,h) that run as one launch (decode_block_kernel: one wave
// per chunk, merged in LDS); larger plans run the split + combine pair.
constexpr int kMaxBlockSplits = 16;
// The automatic plan never picks 9..16 chunks: those would run the 16-wave
// instance (one register set), and 8 chunks on the 8-wave instance (two
// register sets, paired rows at D=64) measured 2-27% faster at every shape
// tried (B1 H12 D64 1K to B16 H32 D128 8K).  Forced split counts still may.
constexpr int kMaxAutoBlockSplits = 8;
// Work units (a (b,h) of a one-launch plan, a (b,h,chunk) of a split plan) that
// met a page id outside [0, num_pages) among the pages their positions use
// (int8k_decode_paged_bad_page_ids).  Such an id reads the last page instead.
__device__ unsigned int g_paged_bad_ids;

// Largest page-id table the paged one-launch kernel stages in LDS (12288 ids);
// longer tables run the paged split + combine pair.
constexpr long long kPagedLdsTableBytes = 48 << 10;

// Plans of at most kMaxBlockSplits chunks run as one launch (decode_block_kernel);
// INT8K_DECODE_BLOCK=0 keeps them on the split + combine pair (read once).
bool use_block_kernel() {
    static const bool on = [] {
        const char* e = std::getenv("INT8K_DECODE_BLOCK");
        return !(e != nullptr && e[0] == '0');
    }();
    return on;
}

inline int env_int(const char* name, int dflt) {
    const char* e = std::getenv(name);
    return e ? std::atoi(e) : dflt;
}

// Defaults measured on MI355X at the BASELINE shapes (B32 H32 D128 8K and
// B8 H32 D64 2K..32K): D=128 — 8 slots, non-temporal K/V loads, ~8192 units
// (two resident rounds at 16 waves/CU); D=64 — 4 slots, non-temporal scale
// loads, ~2048 units (8 chunks per (b,h) at B8 H32: two waves per SIMD);
// its paired-row kernels (plans of up to 8 chunks) load K/V non-temporally
// and the scales as plain loads (ctx 2K-32K: 5-11% faster than the grouped
// rows with non-temporal scales).  Both rotate each unit's starting
// iteration (stagger), which was worth 2-5%.  The INT8K_DECODE_* variables
// override these for tuning sweeps (read once per process).
DecodeTuning tuning_for(int D) {
    static const int e_slots = env_int("INT8K_DECODE_SLOTS", 0);
    static const int e_flags = env_int("INT8K_DECODE_FLAGS", -1);
    static const int e_units = env_int("INT8K_DECODE_TARGET_UNITS", 0);
    static const int e_stagger = env_int("INT8K_DECODE_STAGGER", -1);
    static const int e_pair = env_int("INT8K_DECODE_PAIR_FLAGS", -1);
    DecodeTuning t;
    if (D == 128) t = DecodeTuning{8, kNtKV, 8192, 1, kNtKV};
    else t = DecodeTuning{4, kNtScales, 2048, 1, kNtKV};
    if (e_slots == 4 || e_slots == 8) t.slots = e_slots;
    if (e_flags >= 0) t.flags = e_flags & 3;
    if (e_units > 0) t.target_units = e_units;
    if (e_stagger >= 0) t.stagger = e_stagger;
    if (e_pair >= 0) t.pair_flags = e_pair & 3;
    return t;
}

// Split-count choice: a unit is one wave over one KV chunk of one (b,h);
// aim for tuning.target_units units in total, each chunk a multiple of the
// rows one wave iteration covers.
SplitPlan plan_splits(int BH, int S, int D, int nsplit_req) {
    const DecodeTuning tn = tuning_for(D);
    const int R = rows_per_iter(D, tn.slots);
    const long long max_split = ceil_div(S, R);
    long long ns;
    if (nsplit_req > 0) {
        ns = nsplit_req;
    } else {
        ns = ceil_div(tn.target_units, BH);
        // keep at least 4 iterations per unit unless S is short; an under-filled
        // grid (few (b,h)) may still take up to kMaxAutoBlockSplits short chunks,
        // which the one-launch kernel merges on chip
        const long long by_len = std::max<long long>(
            1, std::max(ceil_div(S, 4LL * R), std::min<long long>(kMaxAutoBlockSplits, ceil_div(S, R))));
        ns = std::min(ns, by_len);
        if (ns > kMaxAutoBlockSplits && ns <= kMaxBlockSplits) ns = kMaxAutoBlockSplits;
    }
    ns = std::max<long long>(1, std::min(ns, max_split));
    long long chunk = round_up((size_t)ceil_div(S, ns), (size_t)R);
    ns = ceil_div(S, chunk);
    return SplitPlan{(int)ns, (int)chunk};
}

struct Int4 {
    int x, y, z, w;
};

__device__ __forceinline__ Int4 load16(const int8_t* p) {
    const int4 v = *reinterpret_cast<const int4*>(p);
    return Int4{v.x, v.y, v.z, v.w};
}

template <bool NT>
__device__ __forceinline__ float load_f32(const float* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

template <bool NT>
__device__ __forceinline__ Int4 load_kv16(const int8_t* p) {
    if constexpr (NT) {
        typedef int v4i __attribute__((ext_vector_type(4)));
        const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
        return Int4{v.x, v.y, v.z, v.w};
    } else {
        return load16(p);
    }
}

__device__ __forceinline__ void fma_bytes(float* acc, int word, float w) {
    acc[0] = fmaf(w, sbyte_to_f32<0>(word), acc[0]);
    acc[1] = fmaf(w, sbyte_to_f32<1>(word), acc[1]);
    acc[2] = fmaf(w, sbyte_to_f32<2>(word), acc[2]);
    acc[3] = fmaf(w, sbyte_to_f32<3>(word), acc[3]);
}

template <int D>
__device__ __forceinline__ int group_sum(int v) {
    if constexpr (D == 128) return group8_sum(v);
    else return group4_sum(v);
}

// Lane t's value of each 4-lane quad, in every lane of the quad (DPP
// quad_perm [t,t,t,t]); t is a compile-time constant after unrolling.
__device__ __forceinline__ float quad_bcast(float x, int t) {
    const int v = __float_as_int(x);
    switch (t) {
        case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x00, 0xF, 0xF, false));
        case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0x55, 0xF, 0xF, false));
        case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xAA, 0xF, 0xF, false));
        default: return __int_as_float(__builtin_amdgcn_mov_dpp(v, 0xFF, 0xF, 0xF, false));
    }
}

// QK^T, online softmax and PV for one wave iteration whose NSLOT rows per
// group are loaded (kv, vv, sk, sv).  MASKED: rows >= j1 get score -inf and
// weight 0 (their loads point at some valid row).  RS: rows between slots
// (2 for paired rows).  QB: sk[0]/sv[0] hold the scale of the lane's own slot
// (lane s of the 4-lane group: slot s), read by the group with quad_bcast.
template <int D, int NS, bool MASKED, int RS = 1, bool QB = false>
__device__ __forceinline__ void decode_math(const Int4 (&kv)[NS], const Int4 (&vv)[NS],
                                            const float (&sk)[NS], const float (&sv)[NS],
                                            int row0, int j1, const Int4& q, float qscale,
                                            float& m, float& l, float* acc) {
    static_assert(!QB || (NS == 4 && D == 64), "quad broadcast: one scale per lane of a group");
    // QK^T: exact int32 dot per row, summed over the LPR lanes of the group.
    float sc[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        int d = __builtin_amdgcn_sdot4(q.x, kv[t].x, 0, false);
        d = __builtin_amdgcn_sdot4(q.y, kv[t].y, d, false);
        d = __builtin_amdgcn_sdot4(q.z, kv[t].z, d, false);
        d = __builtin_amdgcn_sdot4(q.w, kv[t].w, d, false);
        d = group_sum<D>(d);
        const float skt = QB ? quad_bcast(sk[0], t) : sk[t];
        sc[t] = static_cast<float>(d) * qscale * skt;
        if constexpr (MASKED) {
            if (row0 + t * RS >= j1) sc[t] = -INFINITY;
        }
    }

    // Online softmax (log2 domain) for this group's NSLOT rows.
    float mx = sc[0];
#pragma unroll
    for (int t = 1; t < NS; ++t) mx = fmaxf(mx, sc[t]);
    const float m_new = fmaxf(m, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float corr = fast_exp2(m - m_use);
    l *= corr;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] *= corr;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        const float p = fast_exp2(sc[t] - m_use);
        l += p;
        float w = p * (QB ? quad_bcast(sv[0], t) : sv[t]);
        if constexpr (MASKED) {
            if (row0 + t * RS >= j1) w = 0.f;
        }
        fma_bytes(acc + 0, vv[t].x, w);
        fma_bytes(acc + 4, vv[t].y, w);
        fma_bytes(acc + 8, vv[t].z, w);
        fma_bytes(acc + 12, vv[t].w, w);
    }
    m = m_new;
}

// The registers of one wave iteration: NSLOT rows per group of K, V and scales.
template <int NS>
struct IterBuf {
    Int4 kv[NS], vv[NS];
    float sk[NS], sv[NS];
};

// The loads of an unmasked wave iteration whose group rows start at row0 and
// lie RS rows apart.  Paired rows with vector-capable scales (RS == 2 and
// VEC_SCALES) load one scale per lane, slot `sub` (decode_math's QB).
template <int D, int NS, bool VEC_SCALES, int FL, int RS = 1>
__device__ __forceinline__ void load_iter(IterBuf<NS>& b, const int8_t* __restrict__ Kbh,
                                          const int8_t* __restrict__ Vbh,
                                          const float* __restrict__ sKbh,
                                          const float* __restrict__ sVbh, size_t row0, int sub) {
    const int8_t* kp = Kbh + (size_t)row0 * D + sub * 16;
    const int8_t* vp = Vbh + (size_t)row0 * D + sub * 16;
#pragma unroll
    for (int t = 0; t < NS; ++t) b.kv[t] = load_kv16<(FL & kNtKV) != 0>(kp + t * RS * D);
#pragma unroll
    for (int t = 0; t < NS; ++t) b.vv[t] = load_kv16<(FL & kNtKV) != 0>(vp + t * RS * D);
    if constexpr (VEC_SCALES && RS == 2) {
        b.sk[0] = load_f32<(FL & kNtScales) != 0>(sKbh + row0 + 2 * sub);
        b.sv[0] = load_f32<(FL & kNtScales) != 0>(sVbh + row0 + 2 * sub);
    } else if constexpr (VEC_SCALES) {
#pragma unroll
        for (int t = 0; t < NS; t += 4) {
            typedef float v4f __attribute__((ext_vector_type(4)));
            v4f a, c;
            if constexpr ((FL & kNtScales) != 0) {
                a = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(sKbh + row0 + t));
                c = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(sVbh + row0 + t));
            } else {
                a = *reinterpret_cast<const v4f*>(sKbh + row0 + t);
                c = *reinterpret_cast<const v4f*>(sVbh + row0 + t);
            }
            b.sk[t] = a.x; b.sk[t + 1] = a.y; b.sk[t + 2] = a.z; b.sk[t + 3] = a.w;
            b.sv[t] = c.x; b.sv[t + 1] = c.y; b.sv[t + 2] = c.z; b.sv[t + 3] = c.w;
        }
    } else {
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            b.sk[t] = load_f32<(FL & kNtScales) != 0>(sKbh + row0 + t * RS);
            b.sv[t] = load_f32<(FL & kNtScales) != 0>(sVbh + row0 + t * RS);
        }
    }
}

// One wave iteration over NSLOT rows per group.  MASKED handles the last
// partial block of a chunk: rows >= j1 get score -inf and weight 0 (their
// loads are redirected to row j1-1, which is in bounds).  RS: rows between
// slots (2 for paired rows).
template <int D, int NS, bool MASKED, bool VEC_SCALES, int FL, int RS = 1>
__device__ __forceinline__ void decode_iter(
    const int8_t* __restrict__ Kbh, const int8_t* __restrict__ Vbh,
    const float* __restrict__ sKbh, const float* __restrict__ sVbh,
    int row0, int j1, int sub, const Int4& q, float qscale,
    float& m, float& l, float* acc) {
    IterBuf<NS> b;
    if constexpr (!MASKED) {
        load_iter<D, NS, VEC_SCALES, FL, RS>(b, Kbh, Vbh, sKbh, sVbh, row0, sub);
    } else {
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const int r = min(row0 + t * RS, j1 - 1);
            b.kv[t] = load_kv16<(FL & kNtKV) != 0>(Kbh + (size_t)r * D + sub * 16);
            b.vv[t] = load_kv16<(FL & kNtKV) != 0>(Vbh + (size_t)r * D + sub * 16);
            b.sk[t] = load_f32<(FL & kNtScales) != 0>(sKbh + r);
            b.sv[t] = load_f32<(FL & kNtScales) != 0>(sVbh + r);
        }
    }
    decode_math<D, NS, MASKED, RS, (!MASKED && VEC_SCALES && RS == 2)>(
        b.kv, b.vv, b.sk, b.sv, row0, j1, q, qscale, m, l, acc);
}

// Merges the G row-group states of a wave (lanes with equal `sub`) and writes
// the unit's partial state, or with FINAL the normalised fp16 row (a unit that
// saw no rows, L == 0, gives zeros).
template <int D, bool FINAL>
__device__ __forceinline__ void finish_unit(float m, float l, float* acc, int grp, int sub,
                                            int unit, float* __restrict__ part_ml,
                                            float* __restrict__ part_acc,
                                            uint16_t* __restrict__ out) {
    constexpr int LPR = D / 16;
    float M = m;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
    const float f = (m == -INFINITY) ? 0.f : fast_exp2(m - M);
    float L = l * f;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] *= f;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
        L += __shfl_xor(L, off);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] += __shfl_xor(acc[e], off);
    }
    if constexpr (FINAL) {
        if (grp == 0) {
            const float inv = L > 0.f ? 1.f / L : 0.f;
            uint16_t h[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) h[e] = __half_as_ushort(f16_of_f32(acc[e] * inv));
            uint4* dst = reinterpret_cast<uint4*>(out + (size_t)unit * D + sub * 16);
            dst[0] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                                h[6] | (h[7] << 16));
            dst[1] = make_uint4(h[8] | (h[9] << 16), h[10] | (h[11] << 16),
                                h[12] | (h[13] << 16), h[14] | (h[15] << 16));
        }
        return;
    }
    if (grp == 0) {
        float4* dst = reinterpret_cast<float4*>(part_acc + (size_t)unit * D + sub * 16);
        dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
        dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
        dst[2] = make_float4(acc[8], acc[9], acc[10], acc[11]);
        dst[3] = make_float4(acc[12], acc[13], acc[14], acc[15]);
        if (sub == 0) {
            part_ml[2 * (size_t)unit] = M;
            part_ml[2 * (size_t)unit + 1] = L;
        }
    }
}

// Pass 1: one wave per (bh, split); writes the unnormalised partial state,
// or — when the KV sequence is not split (FINAL) — the fp16 output itself.
template <int D, int NS, bool VEC_SCALES, bool FINAL, int FL>
__global__ __launch_bounds__(kBlockThreads) void decode_split_kernel(
    const int8_t* __restrict__ Q, const int8_t* __restrict__ K,
    const int8_t* __restrict__ V, const float* __restrict__ sQ,
    const float* __restrict__ sK, const float* __restrict__ sV,
    float* __restrict__ part_ml, float* __restrict__ part_acc, uint16_t* __restrict__ out,
    int S, int S_cap, int nsplit, int chunk, int units, float qk_scale_log2, int stagger) {
    using G = DecodeGeom<D, NS>;
    const int lane = threadIdx.x & 63;
    const int unit = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (unit >= units) return;  // whole wave exits; no block barrier below
    const int bh = unit / nsplit;
    const int sp = unit - bh * nsplit;
    const int j0 = sp * chunk;
    const int j1 = min(S, j0 + chunk);

    const int sub = lane % G::kLanesPerRow;
    const int grp = lane / G::kLanesPerRow;

    const Int4 q = load16(Q + (size_t)bh * D + sub * 16);
    const float qscale = sQ[bh] * qk_scale_log2;

    // (b,h) rows sit S_cap apart (the cache capacity); the first S are valid
    const int8_t* Kbh = K + (size_t)bh * S_cap * D;
    const int8_t* Vbh = V + (size_t)bh * S_cap * D;
    const float* sKbh = sK + (size_t)bh * S_cap;
    const float* sVbh = sV + (size_t)bh * S_cap;

    float m = -INFINITY, l = 0.f;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;

    // Full iterations, optionally started at a unit-dependent rotation so that
    // concurrent waves do not walk identical address offsets in lockstep.
    const int n_full = (j1 - j0) / G::kRowsPerIter;
    int it = stagger ? (int)(((unsigned)unit * 2654435761u) >> 16) % max(n_full, 1) : 0;
    for (int k = 0; k < n_full; ++k) {
        decode_iter<D, NS, false, VEC_SCALES, FL>(Kbh, Vbh, sKbh, sVbh,
                                                  j0 + it * G::kRowsPerIter + grp * NS, j1, sub,
                                                  q, qscale, m, l, acc);
        it = (it + 1 == n_full) ? 0 : it + 1;
    }
    const int base = j0 + n_full * G::kRowsPerIter;
    if (base < j1)
        decode_iter<D, NS, true, VEC_SCALES, FL>(Kbh, Vbh, sKbh, sVbh, base + grp * NS, j1, sub,
                                                 q, qscale, m, l, acc);

    finish_unit<D, FINAL>(m, l, acc, grp, sub, unit, part_ml, part_acc, out);
}

// The output row of one (b,h) from the merged accumulator (dims lane*D/64 ..
// +D/64 of this lane) and the merged sum L: the fp16 row, or with qout set the
// per-token int8 quantization of that fp16 row (codes and scale as
// int8k_quantize_per_token gives for it).  A whole wave calls it.
template <int D>
__device__ __forceinline__ void emit_row(const float (&acc)[D / 64], float L, int lane, int bh,
                                         uint16_t* __restrict__ out, int8_t* __restrict__ qout,
                                         float* __restrict__ qscale) {
    constexpr int DPL = D / 64;
    const float inv = L > 0.f ? 1.f / L : 0.f;  // no rows at all (empty sequence): zeros
    float y[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) y[i] = __half2float(f16_of_f32(acc[i] * inv));
    if (qout != nullptr) {
        float am = 0.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i) am = fmaxf(am, fabsf(y[i]));
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) am = fmaxf(am, __shfl_xor(am, off));
        const float sc = fmaxf(am, 1e-8f) / 127.f;
#pragma unroll
        for (int i = 0; i < DPL; ++i)
            qout[(size_t)bh * D + lane * DPL + i] = (int8_t)quant_code(y[i], sc);
        if (lane == 0) qscale[bh] = sc;
        return;
    }
#pragma unroll
    for (int i = 0; i < DPL; ++i)
        out[(size_t)bh * D + lane * DPL + i] = __half_as_ushort(__float2half_rn(y[i]));
}

// Pass 2: one wave per bh merges its nsplit partial states into the output row.
template <int D>
__global__ __launch_bounds__(kBlockThreads) void decode_combine_kernel(
    const float* __restrict__ part_ml, const float* __restrict__ part_acc,
    uint16_t* __restrict__ out, int8_t* __restrict__ qout, float* __restrict__ qscale, int BH,
    int nsplit) {
    constexpr int DPL = D / 64;  // dims per lane
    const int lane = threadIdx.x & 63;
    const int bh = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (bh >= BH) return;
    const float* ml = part_ml + 2 * (size_t)bh * nsplit;

    float M = -INFINITY;
    for (int s = lane; s < nsplit; s += 64) M = fmaxf(M, ml[2 * s]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
    const float M_use = (M == -INFINITY) ? 0.f : M;

    float L = 0.f;
    for (int s = lane; s < nsplit; s += 64) L += ml[2 * s + 1] * fast_exp2(ml[2 * s] - M_use);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) L += __shfl_xor(L, off);

    float acc[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) acc[i] = 0.f;
    const float* pa = part_acc + (size_t)bh * nsplit * D + lane * DPL;
    // unrolled so the partial rows of several splits are loaded together (they
    // come from other XCDs' writes, a full memory round trip each)
#pragma unroll 8
    for (int s = 0; s < nsplit; ++s) {
        const float w = fast_exp2(ml[2 * s] - M_use);
#pragma unroll
        for (int i = 0; i < DPL; ++i) acc[i] = fmaf(pa[(size_t)s * D + i], w, acc[i]);
    }
    emit_row<D>(acc, L, lane, bh, out, qout, qscale);
}

// The n_full whole iterations of a wave's chunk, starting at iteration `it` and
// wrapping around.  roff(i): the row offset (from the K/V/scale bases) of the
// group's first row in iteration i; RS: rows between its slots.  PIPE: two
// register sets, iteration k+1's loads issued before iteration k is computed
// (the fences keep the compiler from sinking them).
template <int D, int NS, bool VEC_SCALES, int FL, bool PIPE, int RS, typename RowOff>
__device__ __forceinline__ void walk_iters(const int8_t* __restrict__ K,
                                           const int8_t* __restrict__ V,
                                           const float* __restrict__ sK,
                                           const float* __restrict__ sV, RowOff roff, int n_full,
                                           int it, int sub, const Int4& q, float qscale, float& m,
                                           float& l, float* acc) {
    constexpr bool QB = VEC_SCALES && RS == 2;
    auto nxt = [&](int i) { return (i + 1 == n_full) ? 0 : i + 1; };
    auto load = [&](IterBuf<NS>& b, int i) {
        load_iter<D, NS, VEC_SCALES, FL, RS>(b, K, V, sK, sV, roff(i), sub);
    };
    auto math = [&](const IterBuf<NS>& b) {
        decode_math<D, NS, false, RS, QB>(b.kv, b.vv, b.sk, b.sv, 0, 0, q, qscale, m, l, acc);
    };
    if constexpr (PIPE) {
        IterBuf<NS> ba, bb;
        if (n_full > 0) load(ba, it);
        int k = 0;
        for (; k + 2 < n_full; k += 2) {
            const int it1 = nxt(it);
            load(bb, it1);
            __builtin_amdgcn_sched_barrier(0);
            math(ba);
            it = nxt(it1);
            load(ba, it);
            __builtin_amdgcn_sched_barrier(0);
            math(bb);
        }
        if (n_full - k == 2) {
            load(bb, nxt(it));
            __builtin_amdgcn_sched_barrier(0);
            math(ba);
            math(bb);
        } else if (n_full - k == 1) {
            math(ba);
        }
    } else {
        for (int k = 0; k < n_full; ++k) {
            IterBuf<NS> b;
            load(b, it);
            math(b);
            it = nxt(it);
        }
    }
}

// The end of a one-launch block: each wave merges its row groups (lanes with
// equal `sub`) and leaves (M, L, acc[D]) in LDS; wave 0 merges the nw chunk
// states with the log-sum-exp rule, as decode_combine_kernel, and writes the
// row.  Every wave of the block calls it (it holds the block's barrier).
template <int D, int MAXW>
__device__ __forceinline__ void merge_block(float m, float l, float* acc, int lane, int grp,
                                            int sub, int w, int nw, int bh,
                                            float (&s_ml)[MAXW][2], float (&s_acc)[MAXW][D],
                                            uint16_t* __restrict__ out,
                                            int8_t* __restrict__ qout,
                                            float* __restrict__ qscale) {
    constexpr int LPR = D / 16;
    float M = m;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
    const float f = (m == -INFINITY) ? 0.f : fast_exp2(m - M);
    float Lw = l * f;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] *= f;
#pragma unroll
    for (int off = LPR; off < 64; off <<= 1) {
        Lw += __shfl_xor(Lw, off);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] += __shfl_xor(acc[e], off);
    }
    if (grp == 0) {
        float4* dst = reinterpret_cast<float4*>(&s_acc[w][sub * 16]);
        dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
        dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
        dst[2] = make_float4(acc[8], acc[9], acc[10], acc[11]);
        dst[3] = make_float4(acc[12], acc[13], acc[14], acc[15]);
        if (sub == 0) {
            s_ml[w][0] = M;
            s_ml[w][1] = Lw;
        }
    }
    __syncthreads();
    if (w != 0) return;
    constexpr int DPL = D / 64;
    float Mall = -INFINITY;
    for (int c = 0; c < nw; ++c) Mall = fmaxf(Mall, s_ml[c][0]);
    const float M_use = (Mall == -INFINITY) ? 0.f : Mall;
    float L = 0.f;
    float o[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[i] = 0.f;
    for (int c = 0; c < nw; ++c) {
        const float wt = fast_exp2(s_ml[c][0] - M_use);
        L += s_ml[c][1] * wt;
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[i] = fmaf(s_acc[c][lane * DPL + i], wt, o[i]);
    }
    emit_row<D>(o, L, lane, bh, out, qout, qscale);
}

// One launch for plans of at most kMaxBlockSplits chunks per (b,h): block bh
// runs one wave per chunk (blockDim.x / 64 waves), each wave walks its chunk as
// the split kernel does, merges its row groups and leaves (m, l, acc[D]) in
// LDS; wave 0 then merges the chunks with the log-sum-exp rule and writes the
// row.  No partial state leaves the chip and there is no second launch.
// MAXW: the most waves the instance is launched with (8 or kMaxBlockSplits).
// The 8-wave instance has twice the registers per wave, which lets it keep the
// next iteration's loads in flight (a second register set, two_sets) while the
// current one computes: at 4 slots a short chunk is only a few dependent load
// rounds, so their latency would show; at D = 128 with 8 slots (204 VGPRs, two
// waves per SIMD) the stream then runs at fewer waves per CU with the same
// bytes in flight, which the HBM read rate prefers.
template <int D, int NS, bool VEC_SCALES, int FL, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void decode_block_kernel(
    const int8_t* __restrict__ Q, const int8_t* __restrict__ K,
    const int8_t* __restrict__ V, const float* __restrict__ sQ,
    const float* __restrict__ sK, const float* __restrict__ sV, uint16_t* __restrict__ out,
    int8_t* __restrict__ qout, float* __restrict__ qscale, int S, int S_cap, int chunk,
    float qk_scale_log2, int stagger) {
    using G = DecodeGeom<D, NS>;
    constexpr int LPR = D / 16;
    __shared__ float s_ml[MAXW][2];
    __shared__ __align__(16) float s_acc[MAXW][D];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    const int bh = blockIdx.x;
    const int j0 = w * chunk;
    const int j1 = min(S, j0 + chunk);
    const int sub = lane % LPR;
    const int grp = lane / LPR;

    const Int4 q = load16(Q + (size_t)bh * D + sub * 16);
    const float qscale_l = sQ[bh] * qk_scale_log2;
    const int8_t* Kbh = K + (size_t)bh * S_cap * D;
    const int8_t* Vbh = V + (size_t)bh * S_cap * D;
    const float* sKbh = sK + (size_t)bh * S_cap;
    const float* sVbh = sV + (size_t)bh * S_cap;

    float m = -INFINITY, l = 0.f;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    const int n_full = max(0, j1 - j0) / G::kRowsPerIter;
    const unsigned unit = (unsigned)bh * (unsigned)nw + (unsigned)w;
    const int it = stagger ? (int)((unit * 2654435761u) >> 16) % max(n_full, 1) : 0;
    constexpr bool PAIRED = paired_rows(D, NS, MAXW);
    constexpr int RS = PAIRED ? 2 : 1;
    const int g0 = group_row0<PAIRED, NS>(grp);
    walk_iters<D, NS, VEC_SCALES, FL, two_sets(D, NS, MAXW), RS>(
        Kbh, Vbh, sKbh, sVbh, [&](int i) { return (size_t)(j0 + i * G::kRowsPerIter + g0); },
        n_full, it, sub, q, qscale_l, m, l, acc);
    const int base = j0 + n_full * G::kRowsPerIter;
    if (base < j1)
        decode_iter<D, NS, true, VEC_SCALES, FL, RS>(Kbh, Vbh, sKbh, sVbh, base + g0, j1, sub,
                                                     q, qscale_l, m, l, acc);
    merge_block<D, MAXW>(m, l, acc, lane, grp, sub, w, nw, bh, s_ml, s_acc, out, qout, qscale);
}

// Paged one-launch variant for plans of up to 8 chunks per (b,h): the block
// of (b,h) first copies sequence b's page ids (the first n_tab, clamped to
// [0, num_pages) as in decode_paged_kernel) into LDS, so that each
// iteration's row offset is an LDS read instead of a global load in front of
// its K/V loads; then it walks and merges its chunks as decode_block_kernel.
template <int D, int NS, bool VEC_SCALES, int FL, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void decode_paged_block_kernel(
    const int8_t* __restrict__ Q, const int8_t* __restrict__ Kp,
    const int8_t* __restrict__ Vp, const float* __restrict__ sQ,
    const float* __restrict__ sKp, const float* __restrict__ sVp,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    uint16_t* __restrict__ out, int8_t* __restrict__ qout, float* __restrict__ qscale, int H,
    int num_pages, int log2_page, int max_pages, int n_tab, int chunk, float qk_scale_log2,
    int stagger) {
    using G = DecodeGeom<D, NS>;
    constexpr int LPR = D / 16;
    extern __shared__ int s_pages[];
    __shared__ float s_ml[MAXW][2];
    __shared__ __align__(16) float s_acc[MAXW][D];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int nw = blockDim.x >> 6;
    // With 16-token pages a head's scales in a page are 64 bytes, and heads 2k
    // and 2k+1 share one 128-byte line.  Blocks go to the 8 XCDs in turn, so
    // with 16 | gridDim.x block i of XCD x takes head pair 8 (i / 2) + x: the
    // pair's two heads run at adjacent slots of one XCD (one L2) and walk their
    // pages in the same order (one stagger), and the line is fetched once.
    const bool pair = log2_page < 5 && (gridDim.x & 15) == 0;
    int bh = blockIdx.x;
    if (pair) {
        const int x = bh & 7, i = bh >> 3;
        bh = ((((i >> 1) << 3) + x) << 1) + (i & 1);
    }
    const int b = bh / H, hh = bh - b * H;
    const int page = 1 << log2_page;
    const int32_t* table = block_tables + (size_t)b * max_pages;
    const int len = min(context_lens[b], n_tab << log2_page);
    const int used = (len + page - 1) >> log2_page;  // entries past it are never read
    bool bad = false;
    for (int i = threadIdx.x; i < n_tab; i += blockDim.x) {
        const int id = table[i];
        bad |= i < used && (unsigned)id >= (unsigned)num_pages;
        s_pages[i] = (int)min((unsigned)id, (unsigned)(num_pages - 1));
    }
    if (__syncthreads_or(bad) && threadIdx.x == 0)
        __hip_atomic_fetch_add(&g_paged_bad_ids, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int j0 = w * chunk;
    const int j1 = min(len, j0 + chunk);
    const int sub = lane % LPR;
    const int grp = lane / LPR;
    const Int4 q = load16(Q + (size_t)bh * D + sub * 16);
    const float qscale_l = sQ[bh] * qk_scale_log2;
    // row offset (in rows of the page arrays) of position r of this head
    auto row_off = [&](int r) -> size_t {
        return ((size_t)s_pages[r >> log2_page] * H + hh) * page + (r & (page - 1));
    };

    float m = -INFINITY, l = 0.f;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    const int n_full = max(0, j1 - j0) / G::kRowsPerIter;
    const unsigned unit = (unsigned)(pair ? bh >> 1 : bh) * (unsigned)nw + (unsigned)w;
    const int it = stagger ? (int)((unit * 2654435761u) >> 16) % max(n_full, 1) : 0;
    // a group's rows (NS-aligned, or the 8-aligned pair block) share one page
    constexpr bool PAIRED = paired_rows(D, NS, MAXW);
    constexpr int RS = PAIRED ? 2 : 1;
    const int g0 = group_row0<PAIRED, NS>(grp);
    walk_iters<D, NS, VEC_SCALES, FL, two_sets(D, NS, MAXW), RS>(
        Kp, Vp, sKp, sVp, [&](int i) { return row_off(j0 + i * G::kRowsPerIter + g0); },
        n_full, it, sub, q, qscale_l, m, l, acc);
    const int base = j0 + n_full * G::kRowsPerIter;
    if (base < j1) {
        const int row0 = base + g0;
        IterBuf<NS> bt;
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const size_t r = row_off(min(row0 + t * RS, j1 - 1));
            bt.kv[t] = load_kv16<(FL & kNtKV) != 0>(Kp + r * D + sub * 16);
            bt.vv[t] = load_kv16<(FL & kNtKV) != 0>(Vp + r * D + sub * 16);
            bt.sk[t] = load_f32<(FL & kNtScales) != 0>(sKp + r);
            bt.sv[t] = load_f32<(FL & kNtScales) != 0>(sVp + r);
        }
        decode_math<D, NS, true, RS>(bt.kv, bt.vv, bt.sk, bt.sv, row0, j1, q, qscale_l, m, l,
                                     acc);
    }
    merge_block<D, MAXW>(m, l, acc, lane, grp, sub, w, nw, bh, s_ml, s_acc, out, qout, qscale);
}

// Paged variant of pass 1.  Unit = (b, h, split) as above, over positions
// [j0, j1) of sequence b (j1 <= context_lens[b]).  A group's NSLOT rows are
// NSLOT-aligned and page_size is a multiple of NSLOT, so they sit in one
// page: one table lookup per group per iteration, then the same immediate
// slot offsets as the contiguous kernel.  Page p of head h holds
// K/V [p][h][page_size][D] and scales [p][h][page_size].  FL: the
// non-temporal load flags of the contiguous kernel's tuning for this D.
// VEC_SCALES: a group's NS scales load as 16-byte vectors (its rows are
// NS-aligned inside one page; needs 16-byte aligned scale arrays).
template <int D, int NS, bool FINAL, int FL, bool VEC_SCALES>
__global__ __launch_bounds__(kBlockThreads) void decode_paged_kernel(
    const int8_t* __restrict__ Q, const int8_t* __restrict__ Kp,
    const int8_t* __restrict__ Vp, const float* __restrict__ sQ,
    const float* __restrict__ sKp, const float* __restrict__ sVp,
    const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens,
    float* __restrict__ part_ml, float* __restrict__ part_acc, uint16_t* __restrict__ out,
    int H, int num_pages, int log2_page, int max_pages, int nsplit, int chunk, int units,
    float qk_scale_log2, int stagger) {
    using G = DecodeGeom<D, NS>;
    const int lane = threadIdx.x & 63;
    const int unit = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    if (unit >= units) return;  // whole wave exits; no block barrier below
    const int bh = unit / nsplit;
    const int sp = unit - bh * nsplit;
    const int b = bh / H, hh = bh - b * H;
    const int page = 1 << log2_page;
    const int len = min(context_lens[b], max_pages << log2_page);
    const int j0 = sp * chunk;
    const int j1 = min(len, j0 + chunk);

    const int sub = lane % G::kLanesPerRow;
    const int grp = lane / G::kLanesPerRow;
    const Int4 q = load16(Q + (size_t)bh * D + sub * 16);
    const float qscale = sQ[bh] * qk_scale_log2;
    const int32_t* table = block_tables + (size_t)b * max_pages;
    // element offset of row r of this head (an id outside [0, num_pages) reads the last page
    // and is counted)
    bool bad = false;
    auto row_off = [&](int r) -> size_t {
        const int id = table[r >> log2_page];
        bad |= (unsigned)id >= (unsigned)num_pages;
        const int pg = min((unsigned)id, (unsigned)(num_pages - 1));
        return ((size_t)pg * H + hh) * page + (r & (page - 1));
    };

    float m = -INFINITY, l = 0.f;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    const int n_full = max(0, j1 - j0) / G::kRowsPerIter;
    // Iterations start at a unit-dependent rotation (stagger), and the page id of
    // the next iteration is looked up while the current one computes, so the
    // table load is not a dependent load in front of every iteration's K/V loads.
    int it = stagger ? (int)(((unsigned)unit * 2654435761u) >> 16) % max(n_full, 1) : 0;
    size_t r_next = n_full > 0 ? row_off(j0 + it * G::kRowsPerIter + grp * NS) : 0;
    for (int k = 0; k < n_full; ++k) {
        const int row0 = j0 + it * G::kRowsPerIter + grp * NS;
        const size_t r0 = r_next;
        it = (it + 1 == n_full) ? 0 : it + 1;
        if (k + 1 < n_full) r_next = row_off(j0 + it * G::kRowsPerIter + grp * NS);
        const int8_t* kp = Kp + r0 * D + sub * 16;
        const int8_t* vp = Vp + r0 * D + sub * 16;
        Int4 kv[NS], vv[NS];
        float sk[NS], sv[NS];
#pragma unroll
        for (int t = 0; t < NS; ++t) kv[t] = load_kv16<(FL & kNtKV) != 0>(kp + t * D);
#pragma unroll
        for (int t = 0; t < NS; ++t) vv[t] = load_kv16<(FL & kNtKV) != 0>(vp + t * D);
        if constexpr (VEC_SCALES) {
#pragma unroll
            for (int t = 0; t < NS; t += 4) {
                typedef float v4f __attribute__((ext_vector_type(4)));
                v4f a, b;
                if constexpr ((FL & kNtScales) != 0) {
                    a = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(sKp + r0 + t));
                    b = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(sVp + r0 + t));
                } else {
                    a = *reinterpret_cast<const v4f*>(sKp + r0 + t);
                    b = *reinterpret_cast<const v4f*>(sVp + r0 + t);
                }
                sk[t] = a.x; sk[t + 1] = a.y; sk[t + 2] = a.z; sk[t + 3] = a.w;
                sv[t] = b.x; sv[t + 1] = b.y; sv[t + 2] = b.z; sv[t + 3] = b.w;
            }
        } else {
#pragma unroll
            for (int t = 0; t < NS; ++t) {
                sk[t] = load_f32<(FL & kNtScales) != 0>(sKp + r0 + t);
                sv[t] = load_f32<(FL & kNtScales) != 0>(sVp + r0 + t);
            }
        }
        decode_math<D, NS, false>(kv, vv, sk, sv, row0, j1, q, qscale, m, l, acc);
    }
    const int base = j0 + n_full * G::kRowsPerIter;
    if (base < j1) {
        const int row0 = base + grp * NS;
        Int4 kv[NS], vv[NS];
        float sk[NS], sv[NS];
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const size_t r = row_off(min(row0 + t, j1 - 1));
            kv[t] = load_kv16<(FL & kNtKV) != 0>(Kp + r * D + sub * 16);
            vv[t] = load_kv16<(FL & kNtKV) != 0>(Vp + r * D + sub * 16);
            sk[t] = load_f32<(FL & kNtScales) != 0>(sKp + r);
            sv[t] = load_f32<(FL & kNtScales) != 0>(sVp + r);
        }
        decode_math<D, NS, true>(kv, vv, sk, sv, row0, j1, q, qscale, m, l, acc);
    }
    if (__ballot(bad) != 0 && lane == 0)
        __hip_atomic_fetch_add(&g_paged_bad_ids, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    finish_unit<D, FINAL>(m, l, acc, grp, sub, unit, part_ml, part_acc, out);
}

struct DecodeWorkspace {
    float* part_ml;
    float* part_acc;
    size_t bytes;
};

DecodeWorkspace carve(void* ws, long long units, int D) {
    const size_t ml_bytes = round_up((size_t)units * 2 * sizeof(float), kWorkspaceAlign);
    const size_t acc_bytes = round_up((size_t)units * D * sizeof(float), kWorkspaceAlign);
    char* p = static_cast<char*>(ws);
    return DecodeWorkspace{reinterpret_cast<float*>(p), reinterpret_cast<float*>(p + ml_bytes),
                           ml_bytes + acc_bytes};
}

template <int D, int NS, bool VEC, bool FINAL>
void launch_split(int flags, int stagger, dim3 grid, hipStream_t stream, const int8_t* Q,
                  const int8_t* K, const int8_t* V, const float* sQ, const float* sK,
                  const float* sV, const DecodeWorkspace& w, uint16_t* out, int S, int S_cap,
                  const SplitPlan& plan, int units, float qk) {
#define INT8K_SPLIT_LAUNCH(FLV)                                                      \
    decode_split_kernel<D, NS, VEC, FINAL, FLV><<<grid, kBlockThreads, 0, stream>>>( \
        Q, K, V, sQ, sK, sV, w.part_ml, w.part_acc, out, S, S_cap, plan.nsplit,      \
        plan.chunk, units, qk, stagger)
    switch (flags & 3) {
        case 0: INT8K_SPLIT_LAUNCH(0); break;
        case 1: INT8K_SPLIT_LAUNCH(1); break;
        case 2: INT8K_SPLIT_LAUNCH(2); break;
        default: INT8K_SPLIT_LAUNCH(3); break;
    }
#undef INT8K_SPLIT_LAUNCH
}

// The 8-wave instance takes the paired-row load flags where it pairs rows.
template <int D, int NS, bool VEC>
void launch_block(const DecodeTuning& tn, int BH, hipStream_t stream, const int8_t* Q,
                  const int8_t* K, const int8_t* V, const float* sQ, const float* sK,
                  const float* sV, uint16_t* out, int8_t* qout, float* qs, int S, int S_cap,
                  const SplitPlan& plan, float qk) {
    const int stagger = tn.stagger;
    const bool eight = plan.nsplit <= 8;
    const int flags = (eight && paired_rows(D, NS, 8)) ? tn.pair_flags : tn.flags;
#define INT8K_BLOCK_LAUNCH(FLV)                                                               \
    if (eight)                                                                                \
        decode_block_kernel<D, NS, VEC, FLV, 8><<<(unsigned)BH, 64 * plan.nsplit, 0, stream>>>(  \
            Q, K, V, sQ, sK, sV, out, qout, qs, S, S_cap, plan.chunk, qk, stagger);           \
    else                                                                                      \
        decode_block_kernel<D, NS, VEC, FLV, kMaxBlockSplits>                                 \
            <<<(unsigned)BH, 64 * plan.nsplit, 0, stream>>>(Q, K, V, sQ, sK, sV, out, qout, qs, \
                                                            S, S_cap, plan.chunk, qk, stagger)
    switch (flags & 3) {
        case 0: INT8K_BLOCK_LAUNCH(0); break;
        case 1: INT8K_BLOCK_LAUNCH(1); break;
        case 2: INT8K_BLOCK_LAUNCH(2); break;
        default: INT8K_BLOCK_LAUNCH(3); break;
    }
#undef INT8K_BLOCK_LAUNCH
}

template <int D, bool VEC, bool FINAL>
void launch_split_ns(int ns, int flags, int stagger, dim3 grid, hipStream_t stream,
                     const int8_t* Q, const int8_t* K, const int8_t* V, const float* sQ,
                     const float* sK, const float* sV, const DecodeWorkspace& w, uint16_t* out,
                     int S, int S_cap, const SplitPlan& plan, int units, float qk) {
    if (ns == 4)
        launch_split<D, 4, VEC, FINAL>(flags, stagger, grid, stream, Q, K, V, sQ, sK, sV, w, out,
                                       S, S_cap, plan, units, qk);
    else
        launch_split<D, 8, VEC, FINAL>(flags, stagger, grid, stream, Q, K, V, sQ, sK, sV, w, out,
                                       S, S_cap, plan, units, qk);
}

// Where a decode writes its rows: fp16 `f16`, or int8 `q` + per-row scale `qs`.
struct DecodeOut {
    uint16_t* f16;
    int8_t* q;
    float* qs;
};

template <int D>
int launch_decode(const int8_t* Q, const int8_t* K, const int8_t* V, const DecodeOut& o,
                  const float* sQ, const float* sK, const float* sV, int BH, int S, int S_cap,
                  const SplitPlan& plan, const DecodeWorkspace& w, hipStream_t stream) {
    uint16_t* out = o.f16;
    const long long units = (long long)BH * plan.nsplit;
    const float qk_scale_log2 = (1.0f / std::sqrt((float)D)) * kLog2e;
    const dim3 grid((unsigned)ceil_div(units, kWavesPerBlock));
    const bool vec = (S_cap % 4 == 0) && aligned_to(sK, 16) && aligned_to(sV, 16);
    const DecodeTuning tn = tuning_for(D);
    const int ns = tn.slots;
    const int fl = tn.flags;
    const int sg = tn.stagger;
    const int u = (int)units;
    const float qk = qk_scale_log2;
    if (plan.nsplit <= kMaxBlockSplits && use_block_kernel()) {
        // one launch: the chunks of a (b,h) are the waves of one block
        if (ns == 4) {
            if (vec) launch_block<D, 4, true>(tn, BH, stream, Q, K, V, sQ, sK, sV, out, o.q, o.qs, S, S_cap, plan, qk);
            else launch_block<D, 4, false>(tn, BH, stream, Q, K, V, sQ, sK, sV, out, o.q, o.qs, S, S_cap, plan, qk);
        } else {
            if (vec) launch_block<D, 8, true>(tn, BH, stream, Q, K, V, sQ, sK, sV, out, o.q, o.qs, S, S_cap, plan, qk);
            else launch_block<D, 8, false>(tn, BH, stream, Q, K, V, sQ, sK, sV, out, o.q, o.qs, S, S_cap, plan, qk);
        }
        return check_launch("decode_block_kernel");
    }
    // the in-kernel final write is fp16 only; int8 rows always go through the combine
    const bool final_pass = plan.nsplit == 1 && out != nullptr && aligned_to(out, 16);
    if (vec && final_pass)
        launch_split_ns<D, true, true>(ns, fl, sg, grid, stream, Q, K, V, sQ, sK, sV, w, out, S, S_cap, plan, u, qk);
    else if (vec)
        launch_split_ns<D, true, false>(ns, fl, sg, grid, stream, Q, K, V, sQ, sK, sV, w, out, S, S_cap, plan, u, qk);
    else if (final_pass)
        launch_split_ns<D, false, true>(ns, fl, sg, grid, stream, Q, K, V, sQ, sK, sV, w, out, S, S_cap, plan, u, qk);
    else
        launch_split_ns<D, false, false>(ns, fl, sg, grid, stream, Q, K, V, sQ, sK, sV, w, out, S, S_cap, plan, u, qk);
    int st = check_launch("decode_split_kernel");
    if (st != INT8K_OK || final_pass) return st;
    const dim3 gridc((unsigned)ceil_div(BH, kWavesPerBlock));
    decode_combine_kernel<D><<<gridc, kBlockThreads, 0, stream>>>(w.part_ml, w.part_acc, out,
                                                                  o.q, o.qs, BH, plan.nsplit);
    return check_launch("decode_combine_kernel");
}

template <int D>
int launch_decode_paged(const int8_t* Q, const int8_t* Kp, const int8_t* Vp, const DecodeOut& o,
                        const float* sQ, const float* sKp, const float* sVp,
                        const int32_t* tables, const int32_t* lens, int B, int H,
                        int num_pages, int log2_page, int max_pages, const SplitPlan& plan,
                        const DecodeWorkspace& w, hipStream_t stream) {
    uint16_t* out = o.f16;
    const int BH = B * H;
    const long long units = (long long)BH * plan.nsplit;
    const float qk = (1.0f / std::sqrt((float)D)) * kLog2e;
    const dim3 grid((unsigned)ceil_div(units, kWavesPerBlock));
    constexpr int NS = D == 128 ? 8 : 4;
    const bool vec = aligned_to(sKp, 16) && aligned_to(sVp, 16);
    // page ids the chunks can reach, staged in LDS by the one-launch kernel
    const long long n_tab = std::min<long long>(
        max_pages, ceil_div((long long)plan.nsplit * plan.chunk, 1LL << log2_page));
    if (plan.nsplit <= 8 && use_block_kernel() && n_tab * 4 <= kPagedLdsTableBytes) {
        const int st = tuning_for(D).stagger;
        const size_t lds = (size_t)n_tab * 4;
#define INT8K_PAGED_BLOCK(FLV)                                                                 \
    if (vec)                                                                                   \
        decode_paged_block_kernel<D, NS, true, FLV, 8>                                         \
            <<<(unsigned)BH, 64 * plan.nsplit, lds, stream>>>(                                 \
                Q, Kp, Vp, sQ, sKp, sVp, tables, lens, out, o.q, o.qs, H, num_pages, log2_page, \
                max_pages, (int)n_tab, plan.chunk, qk, st);                                     \
    else                                                                                       \
        decode_paged_block_kernel<D, NS, false, FLV, 8>                                        \
            <<<(unsigned)BH, 64 * plan.nsplit, lds, stream>>>(                                 \
                Q, Kp, Vp, sQ, sKp, sVp, tables, lens, out, o.q, o.qs, H, num_pages, log2_page, \
                max_pages, (int)n_tab, plan.chunk, qk, st)
        const DecodeTuning tn = tuning_for(D);
        switch ((paired_rows(D, NS, 8) ? tn.pair_flags : tn.flags) & 3) {
            case 0: INT8K_PAGED_BLOCK(0); break;
            case 1: INT8K_PAGED_BLOCK(1); break;
            case 2: INT8K_PAGED_BLOCK(2); break;
            default: INT8K_PAGED_BLOCK(3); break;
        }
#undef INT8K_PAGED_BLOCK
        return check_launch("decode_paged_block_kernel");
    }
    const bool final_pass = plan.nsplit == 1 && out != nullptr && aligned_to(out, 16);
#define INT8K_PAGED_LAUNCH(FIN, FLV)                                                         \
    if (vec) decode_paged_kernel<D, NS, FIN, FLV, true><<<grid, kBlockThreads, 0, stream>>>( \
        Q, Kp, Vp, sQ, sKp, sVp, tables, lens, w.part_ml, w.part_acc, out, H, num_pages,     \
        log2_page, max_pages, plan.nsplit, plan.chunk, (int)units, qk, tuning_for(D).stagger); \
    else decode_paged_kernel<D, NS, FIN, FLV, false><<<grid, kBlockThreads, 0, stream>>>(   \
        Q, Kp, Vp, sQ, sKp, sVp, tables, lens, w.part_ml, w.part_acc, out, H, num_pages,     \
        log2_page, max_pages, plan.nsplit, plan.chunk, (int)units, qk, tuning_for(D).stagger)
#define INT8K_PAGED_FLAGS(FIN)                          \
    switch (tuning_for(D).flags & 3) {                  \
        case 0: INT8K_PAGED_LAUNCH(FIN, 0); break;      \
        case 1: INT8K_PAGED_LAUNCH(FIN, 1); break;      \
        case 2: INT8K_PAGED_LAUNCH(FIN, 2); break;      \
        default: INT8K_PAGED_LAUNCH(FIN, 3); break;     \
    }
    if (final_pass) {
        INT8K_PAGED_FLAGS(true)
    } else {
        INT8K_PAGED_FLAGS(false)
    }
#undef INT8K_PAGED_FLAGS
#undef INT8K_PAGED_LAUNCH
    int st = check_launch("decode_paged_kernel");
    if (st != INT8K_OK || final_pass) return st;
    const dim3 gridc((unsigned)ceil_div(BH, kWavesPerBlock));
    decode_combine_kernel<D><<<gridc, kBlockThreads, 0, stream>>>(w.part_ml, w.part_acc, out,
                                                                  o.q, o.qs, BH, plan.nsplit);
    return check_launch("decode_combine_kernel");
}

}  // namespace
}  // namespace int8k

using namespace int8k;

extern "C" int int8k_decode_attention_num_splits(int BH, int S, int head_dim, int nsplit) {
    if (BH <= 0 || S <= 0 || (head_dim != 64 && head_dim != 128)) return 0;
    return plan_splits(BH, S, head_dim, nsplit).nsplit;
}

// Workspace a contiguous-cache decode with this plan needs: none when the chunks
// of each (b,h) merge on chip (decode_block_kernel writes no partials), else
// the split kernel's m, l and acc[D] per unit.
static size_t decode_partial_bytes(const SplitPlan& plan, long long BH, int D) {
    if (plan.nsplit <= kMaxBlockSplits && use_block_kernel()) return 0;
    return carve(nullptr, BH * plan.nsplit, D).bytes;
}

extern "C" size_t int8k_decode_attention_workspace_bytes(int BH, int S, int head_dim, int nsplit) {
    if (BH <= 0 || S <= 0 || (head_dim != 64 && head_dim != 128)) return 0;
    return decode_partial_bytes(plan_splits(BH, S, head_dim, nsplit), BH, head_dim);
}

static bool out_ok(const DecodeOut& o) {
    return o.f16 ? aligned_to(o.f16, 2) : (o.q != nullptr && o.qs != nullptr && aligned_to(o.qs, 4));
}

static int decode_impl(const int8_t* Q, const int8_t* K, const int8_t* V, const DecodeOut& out,
                       const float* scale_Q, const float* scale_K, const float* scale_V, int BH,
                       int S, int S_cap, int head_dim, int nsplit, void* workspace,
                       size_t workspace_bytes, void* stream) {
    clear_last_error();
    if (!Q || !K || !V || !(out.f16 || out.q) || !scale_Q || !scale_K || !scale_V)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (BH <= 0 || S <= 0 || S_cap < S || nsplit < 0) return INT8K_ERR_INVALID_ARGUMENT;
    if (head_dim != 64 && head_dim != 128) return INT8K_ERR_UNSUPPORTED;
    if (!out.f16 && !out.qs) return INT8K_ERR_INVALID_ARGUMENT;
    if (!aligned_to(Q, 16) || !aligned_to(K, 16) || !aligned_to(V, 16) ||
        !aligned_to(scale_Q, 4) || !aligned_to(scale_K, 4) || !aligned_to(scale_V, 4) ||
        !out_ok(out))
        return INT8K_ERR_MISALIGNED;
    const SplitPlan plan = plan_splits(BH, S, head_dim, nsplit);
    const long long units = (long long)BH * plan.nsplit;
    if (units >= (1LL << 26)) return INT8K_ERR_UNSUPPORTED;  // 64 work-items per unit, < 2^32
    // the one-launch path reads no workspace: a null or short one is accepted there
    if (decode_partial_bytes(plan, BH, head_dim) > 0) {
        if (!workspace || workspace_bytes < carve(nullptr, units, head_dim).bytes)
            return INT8K_ERR_WORKSPACE;
        if (!aligned_to(workspace, 16)) return INT8K_ERR_MISALIGNED;
    }
    const DecodeWorkspace w = carve(workspace, units, head_dim);
    if (head_dim == 128)
        return launch_decode<128>(Q, K, V, out, scale_Q, scale_K, scale_V, BH, S, S_cap, plan,
                                  w, as_stream(stream));
    return launch_decode<64>(Q, K, V, out, scale_Q, scale_K, scale_V, BH, S, S_cap, plan, w,
                             as_stream(stream));
}

extern "C" int int8k_decode_attention_forward(
    const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int BH, int S, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream) {
    if (!out) return INT8K_ERR_INVALID_ARGUMENT;
    return decode_impl(Q, K, V, DecodeOut{out, nullptr, nullptr}, scale_Q, scale_K, scale_V, BH,
                       S, S, head_dim, nsplit, workspace, workspace_bytes, stream);
}

extern "C" int int8k_decode_attention_forward_quant(
    const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* out_q, float* out_scale,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int BH, int S, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream) {
    if (!out_q || !out_scale) return INT8K_ERR_INVALID_ARGUMENT;
    return decode_impl(Q, K, V, DecodeOut{nullptr, out_q, out_scale}, scale_Q, scale_K, scale_V,
                       BH, S, S, head_dim, nsplit, workspace, workspace_bytes, stream);
}

extern "C" int int8k_decode_attention_forward_cache(
    const int8_t* Q, const int8_t* K_cache, const int8_t* V_cache, uint16_t* out,
    const float* scale_Q, const float* sK_cache, const float* sV_cache,
    int BH, int S, int capacity, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream) {
    if (!out) return INT8K_ERR_INVALID_ARGUMENT;
    return decode_impl(Q, K_cache, V_cache, DecodeOut{out, nullptr, nullptr}, scale_Q, sK_cache,
                       sV_cache, BH, S, capacity, head_dim, nsplit, workspace, workspace_bytes,
                       stream);
}

extern "C" int int8k_decode_attention_forward_cache_quant(
    const int8_t* Q, const int8_t* K_cache, const int8_t* V_cache, int8_t* out_q,
    float* out_scale, const float* scale_Q, const float* sK_cache, const float* sV_cache,
    int BH, int S, int capacity, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream) {
    if (!out_q || !out_scale) return INT8K_ERR_INVALID_ARGUMENT;
    return decode_impl(Q, K_cache, V_cache, DecodeOut{nullptr, out_q, out_scale}, scale_Q,
                       sK_cache, sV_cache, BH, S, capacity, head_dim, nsplit, workspace,
                       workspace_bytes, stream);
}

// The paged kernel always uses 8 slots for D = 128 and 4 for D = 64 (page_size
// is a multiple of both), so its split plan is computed for those slot counts.
static SplitPlan plan_paged(int BH, int max_context, int D, int nsplit_req) {
    const int ns_slots = D == 128 ? 8 : 4;
    const int R = rows_per_iter(D, ns_slots);
    const DecodeTuning tn = tuning_for(D);
    const long long max_split = ceil_div(max_context, R);
    long long ns;
    if (nsplit_req > 0) {
        ns = nsplit_req;
    } else {
        ns = ceil_div(tn.target_units, BH);
        ns = std::min(ns, std::max<long long>(1, ceil_div(max_context, 4LL * R)));
    }
    ns = std::max<long long>(1, std::min(ns, max_split));
    const long long chunk = round_up((size_t)ceil_div(max_context, ns), (size_t)R);
    ns = ceil_div(max_context, chunk);
    return SplitPlan{(int)ns, (int)chunk};
}

extern "C" size_t int8k_decode_attention_paged_workspace_bytes(int B, int H, int max_context,
                                                               int head_dim, int nsplit) {
    if (B <= 0 || H <= 0 || max_context <= 0 || (head_dim != 64 && head_dim != 128)) return 0;
    const long long BH = (long long)B * H;
    if (BH >= (1LL << 31)) return 0;
    const SplitPlan plan = plan_paged((int)BH, max_context, head_dim, nsplit);
    return carve(nullptr, BH * plan.nsplit, head_dim).bytes;
}

extern "C" int int8k_decode_attention_paged_num_splits(int B, int H, int max_context,
                                                       int head_dim, int nsplit) {
    if (B <= 0 || H <= 0 || max_context <= 0 || (head_dim != 64 && head_dim != 128)) return 0;
    const long long BH = (long long)B * H;
    if (BH >= (1LL << 31)) return 0;
    return plan_paged((int)BH, max_context, head_dim, nsplit).nsplit;
}

extern "C" int int8k_decode_paged_bad_page_ids(unsigned int* count) {
    clear_last_error();
    if (!count) return INT8K_ERR_INVALID_ARGUMENT;
    const hipError_t e = hipMemcpyFromSymbol(count, HIP_SYMBOL(g_paged_bad_ids),
                                             sizeof(unsigned int), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        set_last_error("hipMemcpyFromSymbol(g_paged_bad_ids)", e);
        return INT8K_ERR_HIP;
    }
    return INT8K_OK;
}

static int paged_impl(
    const int8_t* Q, const int8_t* K_pages, const int8_t* V_pages, const DecodeOut& out,
    const float* scale_Q, const float* sK_pages, const float* sV_pages,
    const int32_t* block_tables, const int32_t* context_lens,
    int B, int H, int head_dim, int num_pages, int page_size, int max_pages_per_seq,
    int max_context, int nsplit, void* workspace, size_t workspace_bytes, void* stream) {
    clear_last_error();
    if (!Q || !K_pages || !V_pages || !(out.f16 || (out.q && out.qs)) || !scale_Q || !sK_pages ||
        !sV_pages || !block_tables || !context_lens)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (B <= 0 || H <= 0 || num_pages <= 0 || max_pages_per_seq <= 0 || max_context <= 0 ||
        nsplit < 0)
        return INT8K_ERR_INVALID_ARGUMENT;
    if (head_dim != 64 && head_dim != 128) return INT8K_ERR_UNSUPPORTED;
    if (page_size < 16 || page_size > 1024 || (page_size & (page_size - 1)) != 0)
        return INT8K_ERR_UNSUPPORTED;
    if ((long long)max_context > (long long)max_pages_per_seq * page_size)
        return INT8K_ERR_INVALID_ARGUMENT;
    const long long BH = (long long)B * H;
    if ((long long)num_pages * H * page_size * head_dim >= (1LL << 40)) return INT8K_ERR_UNSUPPORTED;
    if (!aligned_to(Q, 16) || !aligned_to(K_pages, 16) || !aligned_to(V_pages, 16) ||
        !aligned_to(scale_Q, 4) || !aligned_to(sK_pages, 4) || !aligned_to(sV_pages, 4) ||
        !aligned_to(block_tables, 4) || !aligned_to(context_lens, 4) || !out_ok(out))
        return INT8K_ERR_MISALIGNED;
    if (BH >= (1LL << 31)) return INT8K_ERR_UNSUPPORTED;
    const SplitPlan plan = plan_paged((int)BH, max_context, head_dim, nsplit);
    const long long units = BH * plan.nsplit;
    if (units >= (1LL << 26)) return INT8K_ERR_UNSUPPORTED;  // 64 work-items per unit, < 2^32
    const DecodeWorkspace w = carve(workspace, units, head_dim);
    if (!workspace || workspace_bytes < w.bytes) return INT8K_ERR_WORKSPACE;
    if (!aligned_to(workspace, 16)) return INT8K_ERR_MISALIGNED;
    int log2_page = 0;
    while ((1 << log2_page) < page_size) ++log2_page;
    if (head_dim == 128)
        return launch_decode_paged<128>(Q, K_pages, V_pages, out, scale_Q, sK_pages, sV_pages,
                                        block_tables, context_lens, B, H, num_pages, log2_page,
                                        max_pages_per_seq, plan, w, as_stream(stream));
    return launch_decode_paged<64>(Q, K_pages, V_pages, out, scale_Q, sK_pages, sV_pages,
                                   block_tables, context_lens, B, H, num_pages, log2_page,
                                   max_pages_per_seq, plan, w, as_stream(stream));
}

extern "C" int int8k_decode_attention_forward_paged(
    const int8_t* Q, const int8_t* K_pages, const int8_t* V_pages, uint16_t* out,
    const float* scale_Q, const float* sK_pages, const float* sV_pages,
    const int32_t* block_tables, const int32_t* context_lens,
    int B, int H, int head_dim, int num_pages, int page_size, int max_pages_per_seq,
    int max_context, int nsplit, void* workspace, size_t workspace_bytes, void* stream) {
    if (!out) return INT8K_ERR_INVALID_ARGUMENT;
    return paged_impl(Q, K_pages, V_pages, DecodeOut{out, nullptr, nullptr}, scale_Q, sK_pages,
                      sV_pages, block_tables, context_lens, B, H, head_dim, num_pages, page_size,
                      max_pages_per_seq, max_context, nsplit, workspace, workspace_bytes, stream);
}

extern "C" int int8k_decode_attention_forward_paged_quant(
    const int8_t* Q, const int8_t* K_pages, const int8_t* V_pages, int8_t* out_q,
    float* out_scale, const float* scale_Q, const float* sK_pages, const float* sV_pages,
    const int32_t* block_tables, const int32_t* context_lens,
    int B, int H, int head_dim, int num_pages, int page_size, int max_pages_per_seq,
    int max_context, int nsplit, void* workspace, size_t workspace_bytes, void* stream) {
    if (!out_q || !out_scale) return INT8K_ERR_INVALID_ARGUMENT;
    return paged_impl(Q, K_pages, V_pages, DecodeOut{nullptr, out_q, out_scale}, scale_Q,
                      sK_pages, sV_pages, block_tables, context_lens, B, H, head_dim, num_pages,
                      page_size, max_pages_per_seq, max_context, nsplit, workspace,
                      workspace_bytes, stream);
}
