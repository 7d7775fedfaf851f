/*
 * int8k.h — C ABI of the MI355X (gfx950) INT8 transformer-inference kernels.
 *
 * Every entry point takes plain device pointers, element counts and an opaque
 * HIP stream (a hipStream_t passed as void*; NULL means the legacy default
 * stream).  Nothing here allocates device memory: operations that need
 * scratch take a caller-owned workspace whose size comes from the matching
 * *_workspace_bytes() query.  Every call returns an int8k_status; launches are
 * asynchronous on the given stream and are checked with hipGetLastError().
 *
 * Numerical contract (shared with the reference L1 launchers cited below):
 *   - per-token symmetric scales: x ~= q * s, s = max(|row|, 1e-8) / 127,
 *     q = round-half-even(x / s) clamped to [-128, 127];
 *   - fp16 means IEEE binary16 stored in uint16_t;
 *   - attention scale 1/sqrt(head_dim), softmax in fp32, output fp16.
 *
 * The entry points replace the raw-pointer C++ launchers that the reference's
 * torch binding forward-declares at kernels/int8_ext.cu:26-70.
 */
#ifndef INT8K_H
#define INT8K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INT8K_ABI_VERSION 1

typedef enum int8k_status {
    INT8K_OK = 0,
    INT8K_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative or zero size, shape mismatch */
    INT8K_ERR_UNSUPPORTED = 2,      /* valid but unsupported configuration (e.g. head_dim) */
    INT8K_ERR_WORKSPACE = 3,        /* workspace missing or smaller than the query says */
    INT8K_ERR_MISALIGNED = 4,       /* a pointer violates the documented alignment */
    INT8K_ERR_HIP = 5               /* the HIP runtime reported an error at launch */
} int8k_status;

/* Human-readable text for a status code (static storage, never NULL). */
const char* int8k_status_string(int status);

/* INT8K_ABI_VERSION of the built library. */
int int8k_abi_version(void);

/* Text of the last HIP error seen by this thread's most recent failing call
 * ("" if none). */
const char* int8k_last_error(void);

/* ------------------------------------------------------------------------ */
/* Split-KV decode attention (seq_q == 1) over a contiguous INT8 KV cache.   */
/*                                                                          */
/* Replaces int8_decode_attention_forward(Q, K, V, out, scale_Q, scale_K,   */
/* scale_V, BH, S, head_dim) — kernels/int8_decode_attention.cu:443-447,     */
/* declared at kernels/int8_ext.cu:33-37.                                    */
/*                                                                          */
/*   Q   int8 [BH, D]        sQ float [BH]                                   */
/*   K,V int8 [BH, S, D]     sK, sV float [BH*S]  (index bh*S + j)           */
/*   out fp16 [BH, D]                                                        */
/*   out[bh] = sum_j softmax_j(q.k_j * sQ*sK_j / sqrt(D)) * (v_j * sV_j)     */
/*                                                                          */
/* D must be 64 or 128 (as the reference binding checks, kernels/int8_ext.cu */
/* :160-161); S >= 1.  Q, K, V must be 16-byte aligned.  nsplit = 0 picks    */
/* the split count automatically (sized for 256 CUs); a positive value       */
/* forces that many KV chunks per (b,h) (clamped to what S allows) — the     */
/* result is independent of it up to fp32 rounding.                          */
/*                                                                          */
/* The workspace holds split partials.  Plans of at most 16 chunks per (b,h) */
/* merge their chunks on chip and need none: the query returns 0 and the    */
/* call accepts a null workspace for them.                                  */
/* ------------------------------------------------------------------------ */
size_t int8k_decode_attention_workspace_bytes(int BH, int S, int head_dim, int nsplit);

int int8k_decode_attention_forward(
    const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int BH, int S, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream);

/* The same decode emitting int8 rows: out_q int8 [BH, D] and out_scale fp32
 * [BH], the per-token quantization of the fp16 rows the call above returns
 * (as int8k_attention_forward_quant for prefill).  Same workspace. */
int int8k_decode_attention_forward_quant(
    const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* out_q, float* out_scale,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int BH, int S, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream);

/* The split count the forward call uses for this shape (after clamping). */
int int8k_decode_attention_num_splits(int BH, int S, int head_dim, int nsplit);

/* int8k_decode_attention_forward without a workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  It allocates nothing: the split partials go to a device array
 * the library holds, INT8K_DECODE_NOALLOC_SCRATCH_BYTES per GPU, from the
 * library's load until the process ends.  A call whose
 * int8k_decode_attention_workspace_bytes() exceeds that size returns
 * INT8K_ERR_WORKSPACE (int8k_last_error() says why) before touching the GPU;
 * plans that merge their chunks on chip need no scratch and are never
 * rejected for size.
 * All calls on one GPU share its array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.  Same
 * arguments, results and alignment as int8k_decode_attention_forward. */
#define INT8K_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)

int int8k_decode_attention_forward_noalloc(
    const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int BH, int S, int head_dim, int nsplit, void* stream);

/* Decode over a preallocated KV cache: K_cache/V_cache int8 [BH, capacity, D],
 * sK_cache/sV_cache fp32 [BH*capacity]; the first S positions of each (b,h)
 * are attended (S <= capacity).  Same math and workspace as
 * int8k_decode_attention_forward, which is the case capacity == S.  No
 * counterpart in the reference (its decode needs a contiguous [B,H,S,D]
 * tensor); pairs with int8k_kv_cache_append. */
int int8k_decode_attention_forward_cache(
    const int8_t* Q, const int8_t* K_cache, const int8_t* V_cache, uint16_t* out,
    const float* scale_Q, const float* sK_cache, const float* sV_cache,
    int BH, int S, int capacity, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream);

/* int8 rows (out_q [BH, D], out_scale [BH]) from the cache decode; see
 * int8k_decode_attention_forward_quant. */
int int8k_decode_attention_forward_cache_quant(
    const int8_t* Q, const int8_t* K_cache, const int8_t* V_cache, int8_t* out_q,
    float* out_scale, const float* scale_Q, const float* sK_cache, const float* sV_cache,
    int BH, int S, int capacity, int head_dim, int nsplit,
    void* workspace, size_t workspace_bytes, void* stream);

/* Decode over a paged INT8 KV cache (no counterpart in the reference, whose
 * decode is contiguous only — kernels/int8_decode_attention.cu:443-547; this
 * is the serving layout a page-table caller uses).
 *
 *   Q int8 [B, H, D], scale_Q fp32 [B*H]
 *   K_pages / V_pages int8 [num_pages, H, page_size, D]
 *   sK_pages / sV_pages fp32 [num_pages, H, page_size]
 *   block_tables int32 [B, max_pages_per_seq]: page of positions
 *       [i*page_size, (i+1)*page_size) of sequence b is block_tables[b][i]
 *   context_lens int32 [B]: sequence b attends to positions 0 .. len-1,
 *       1 <= len <= max_context (a length of 0 gives a zero output row)
 *   out fp16 [B, H, D]
 *
 * Same math as int8k_decode_attention_forward per (b, h) over the gathered
 * positions.  page_size must be a power of two in [16, 1024];
 * max_context <= max_pages_per_seq * page_size.  A page id outside
 * [0, num_pages) reads page num_pages-1, so a corrupt table reads wrong pages
 * rather than memory outside the cache, and is counted (see
 * int8k_decode_paged_bad_page_ids).  nsplit as for the contiguous call, planned on
 * max_context; the workspace comes from
 * int8k_decode_attention_paged_workspace_bytes. */
size_t int8k_decode_attention_paged_workspace_bytes(int B, int H, int max_context,
                                                    int head_dim, int nsplit);

/* Chunks per (b, h) the paged call plans for these arguments (0 if they are
 * invalid).  Plans of up to 8 chunks whose page-id table fits 48 KiB run as
 * one launch; larger ones as a split kernel plus a combine kernel. */
int int8k_decode_attention_paged_num_splits(int B, int H, int max_context, int head_dim,
                                            int nsplit);

int int8k_decode_attention_forward_paged(
    const int8_t* Q, const int8_t* K_pages, const int8_t* V_pages, uint16_t* out,
    const float* scale_Q, const float* sK_pages, const float* sV_pages,
    const int32_t* block_tables, const int32_t* context_lens,
    int B, int H, int head_dim, int num_pages, int page_size, int max_pages_per_seq,
    int max_context, int nsplit, void* workspace, size_t workspace_bytes, void* stream);

/* Diagnostics of the paged calls: *count receives how many work units, on the
 * current device since the library was loaded, met a page id outside
 * [0, num_pages) among the table entries their positions use (entries past a
 * sequence's length are never read and never counted).  A unit is a (b, h) for
 * plans of up to 8 chunks and a (b, h, chunk) for larger ones, so one bad entry
 * counts at least once per head of its sequence.  Synchronises with the device.
 * No counterpart in the reference, whose decode has no page table. */
int int8k_decode_paged_bad_page_ids(unsigned int* count);

/* int8 rows (out_q [B, H, D], out_scale [B*H]) from the paged decode; see
 * int8k_decode_attention_forward_quant. */
int int8k_decode_attention_forward_paged_quant(
    const int8_t* Q, const int8_t* K_pages, const int8_t* V_pages, int8_t* out_q,
    float* out_scale, const float* scale_Q, const float* sK_pages, const float* sV_pages,
    const int32_t* block_tables, const int32_t* context_lens,
    int B, int H, int head_dim, int num_pages, int page_size, int max_pages_per_seq,
    int max_context, int nsplit, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* INT8 prefill attention (seq_q == seq_kv).                                 */
/*                                                                          */
/* Replaces int8_attention_forward(Q, K, V, out, scale_Q, scale_K, scale_V,  */
/* batch, heads, seq_len, head_dim) — kernels/int8_attention.cu:926-929,     */
/* declared at kernels/int8_ext.cu:27-31 — and adds `causal` (the reference  */
/* is non-causal only; causal = 0 reproduces it).                            */
/*                                                                          */
/*   Q, K, V int8 [batch, heads, seq_len, head_dim]                          */
/*   scale_Q/K/V fp32 [batch*heads*seq_len] (per token)                      */
/*   out fp16 [batch, heads, seq_len, head_dim]                              */
/*   s_ij = (q_i.k_j) sQ_i sK_j / sqrt(D);  out_i = sum_j softmax_j(s) v_j sV_j*/
/*   causal: key j visible to query i iff j <= i.                            */
/* head_dim 1..512; seq_len >= 1.  Multiples of 16 up to 256 run the MFMA   */
/* kernel (Q, K, V 16-byte aligned, out 8-byte aligned); other head dims run */
/* a generic kernel (no alignment beyond the element size), as the          */
/* reference's scalar fallback does (kernels/int8_attention.cu:65-157).      */
/*                                                                          */
/* flags: INT8K_ATTN_CAUSAL (1) = the causal mask (0 reproduces the          */
/* reference); INT8K_ATTN_OUT_BSHD (2) = out in [batch, seq_len, heads,      */
/* head_dim] order, the row order the output projection reads, so no         */
/* transpose copy is needed between them (the reference block makes one in  */
/* PyTorch, bench/bench_block.py:121-124).  Other bits are an invalid        */
/* argument.                                                                 */
/* ------------------------------------------------------------------------ */
#define INT8K_ATTN_CAUSAL 1
#define INT8K_ATTN_OUT_BSHD 2

int int8k_attention_forward(
    const int8_t* Q, const int8_t* K, const int8_t* V, uint16_t* out,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int batch, int heads, int seq_len, int head_dim, int flags, void* stream);

/* Attention output emitted as the next INT8 stage's input: out_q int8
 * [batch, heads, seq_len, head_dim] and out_scale fp32 [batch*heads*seq_len],
 * the per-token quantization (int8k_quantize_per_token) of the fp16 rows
 * int8k_attention_forward returns, byte for byte, without their round trip
 * through memory.  The attention-output producer fusion the reference names
 * as its next lever (OPTIMIZATION.md:241-246; its callers quantize in
 * PyTorch, bench/bench_block.py:59-63); no counterpart in its kernels.
 * out_q and out_scale 4-byte aligned; otherwise as int8k_attention_forward,
 * flags included (with INT8K_ATTN_OUT_BSHD, out_q is [batch, seq_len, heads,
 * head_dim] and out_scale [batch*seq_len*heads] in that order). */
int int8k_attention_forward_quant(
    const int8_t* Q, const int8_t* K, const int8_t* V, int8_t* out_q, float* out_scale,
    const float* scale_Q, const float* scale_K, const float* scale_V,
    int batch, int heads, int seq_len, int head_dim, int flags, void* stream);

/* ------------------------------------------------------------------------ */
/* INT8 MLP: Linear -> GELU(tanh) -> Linear with dynamic per-token requant.  */
/*                                                                          */
/*   x  int8 [T, d_model]    W1 int8 [d_model, d_ff]   W2 int8 [d_ff, d_model]*/
/*   (or, with INT8K_MLP_WEIGHTS_PREPACKED, W1T [d_ff, d_model] and          */
/*    W2T [d_model, d_ff] from int8k_transpose_int8_weights)                 */
/*   scale_x  [T] or [1]; scale_W1 [d_ff] or [1]; scale_W2 [d_model] or [1]   */
/*   (n_scale_* gives the length; 1 broadcasts); bias1 [d_ff] fp32 or NULL,  */
/*   added before GELU.                                                      */
/*   out int8 [T, d_model]; out_scale fp32 [T] (per-token output) or [1]     */
/*   with INT8K_MLP_OUT_PER_TENSOR.                                          */
/*                                                                          */
/* One entry point covers the reference's four MLP launchers                 */
/* (declared at kernels/int8_ext.cu:39-68):                                  */
/*   int8_mlp_forward            (kernels/int8_mlp.cu:1231-1240):            */
/*       n_scale_* = 1, INT8K_MLP_OUT_PER_TENSOR;                            */
/*   int8_mlp_forward_per_channel (kernels/int8_mlp.cu:1248-1258):           */
/*       n_scale_x = T, n_scale_W1 = d_ff, n_scale_W2 = d_model;             */
/*   int8_mlp_forward_per_channel_bias (kernels/int8_mlp.cu:1267-1279):      */
/*       as above with bias1;                                                */
/*   int8_mlp_forward_prepacked  (kernels/int8_mlp.cu:1304-1314):            */
/*       INT8K_MLP_WEIGHTS_PREPACKED | INT8K_MLP_OUT_PER_TENSOR.             */
/* int8_mlp_get_output_scale (kernels/int8_mlp.cu:1317-1322) has no          */
/* counterpart: the scale is written to out_scale on the stream instead of   */
/* being read back from a library global.                                    */
/* d_model and d_ff must be multiples of 16; T is arbitrary.  x, W1, W2 must */
/* be 16-byte aligned.  A GEMM operand (x, W1, W2 or the T x d_ff hidden) of */
/* 4 GiB or more on the large-grid kernels returns INT8K_ERR_UNSUPPORTED     */
/* from the argument checks, before anything is launched.                   */
/* ------------------------------------------------------------------------ */
#define INT8K_MLP_WEIGHTS_PREPACKED 1
#define INT8K_MLP_OUT_PER_TENSOR 2
/* Where a GEMM runs on the 256 x 256 tiled kernel (T * d_ff or T * d_model
 * above 2^23, d_ff and d_model up to 32768), its epilogue finishes the
 * per-token requantization: the tiles of a 256-row stripe exchange their row
 * maxima through the workspace, and neither the fp16 hidden nor the fp16
 * output reaches memory.  The codes are those of the separate pass (fp16 rows
 * + requant), byte for byte.  This flag keeps the separate pass (no
 * counterpart in the reference; for comparison and measurement). */
#define INT8K_MLP_SEPARATE_REQUANT 4

size_t int8k_mlp_workspace_bytes(int T, int d_model, int d_ff, int flags);

/* Diagnostics of the fused requantization: *count receives how many tiles, on
 * the current device since the library was loaded, stopped waiting for their
 * stripe's row maxima (a bounded wait that gives up after ~0.67 s and then
 * uses the maxima that have arrived).  It stays 0 when every tile of a stripe
 * can be resident at once, which the launch order provides on MI355X.
 * Synchronises with the device.  No counterpart in the reference. */
int int8k_mlp_sync_timeouts(unsigned int* count);

int int8k_mlp_forward(
    const int8_t* x, const int8_t* W1, const int8_t* W2, int8_t* out,
    const float* scale_x, int n_scale_x, const float* scale_W1, int n_scale_W1,
    const float* scale_W2, int n_scale_W2, const float* bias1, float* out_scale,
    int T, int d_model, int d_ff, int flags,
    void* workspace, size_t workspace_bytes, void* stream);

/* W1 [d_model, d_ff] -> W1T [d_ff, d_model]; W2 [d_ff, d_model] -> W2T     */
/* [d_model, d_ff].  Replaces transpose_int8_weights                         */
/* (kernels/int8_mlp.cu:1288-1297, declared kernels/int8_ext.cu:59-62).      */
int int8k_transpose_int8_weights(const int8_t* W1, const int8_t* W2, int8_t* W1T, int8_t* W2T,
                                 int d_model, int d_ff, void* stream);

/* Raw C[M,N] = A[M,K] . Bt[N,K]^T with exact int32 accumulation (the MLP's */
/* GEMM core, kernels/int8_mlp.cu:242-310, exposed so its accumulators can   */
/* be checked bit-exactly).  K % 16 == 0; A, Bt 16-byte aligned; M*K and    */
/* N*K below 4 GiB (else INT8K_ERR_UNSUPPORTED, before any launch).         */
int int8k_gemm_i8_i32(const int8_t* A, const int8_t* Bt, int32_t* C, int M, int N, int K,
                      void* stream);

/* ------------------------------------------------------------------------ */
/* Quantization.                                                            */
/* ------------------------------------------------------------------------ */
typedef enum int8k_dtype {
    INT8K_DTYPE_F16 = 0,
    INT8K_DTYPE_BF16 = 1,
    INT8K_DTYPE_F32 = 2
} int8k_dtype;

/* Per-tensor fp16 -> int8: *d_scale (device) receives max(amax,1e-8)/127 and
 * output[i] = rn(clamp(input[i] / scale)).  Replaces quantize_fp16_to_int8
 * (kernels/quant_utils.cu:56-69, declared kernels/int8_common.cuh:51-55); the
 * reference returns scale 0 and code -128 for an all-zero input, this one
 * guards amax with 1e-8 as the reference's Python quantizers do. */
int int8k_quantize_fp16_to_int8(const uint16_t* input, int8_t* output, float* d_scale,
                                long long n, void* stream);

/* output[i] = fp16(input[i] * scale) with a host-side scale.  Replaces
 * dequantize_int8_to_fp16 (kernels/quant_utils.cu:72-77). */
int int8k_dequantize_int8_to_fp16(const int8_t* input, uint16_t* output, float scale,
                                  long long n, void* stream);

/* Per-token (row) quantization of x [rows, cols] (fp16, bf16 or fp32):
 * scales[r] = max(max_c |x[r,c]|, 1e-8)/127, q = rn(clamp(x / s, -128, 127)) —
 * bit-identical to the reference's Python quantizer
 * (validation/check_decode.py:42-47), which every caller runs before the
 * attention and MLP ops.  No C counterpart in the reference. */
int int8k_quantize_per_token(const void* x, int dtype, int8_t* q, float* scales,
                             long long rows, int cols, void* stream);

/* Per-token (row) dequantization of q [rows, cols] int8 with scales [rows]
 * into y [rows, cols] of `dtype`: y = T(float(q) * s_row), T the rounding to
 * the dtype applied to the fp32 product (PyTorch's
 * `(q.float() * s[:, None]).to(dtype)`, two roundings); with a non-NULL
 * residual [rows, cols] of the same dtype, y = T(float(residual) + that) (the
 * residual add of a transformer block).  The consumer side of the INT8 MLP
 * output (int8 + per-token scale).  No counterpart in the reference (its
 * callers dequantize in PyTorch, bench/bench_block.py:113, 126-127). */
int int8k_dequantize_per_token(const int8_t* q, const float* scales, int dtype,
                               const void* residual, void* y, long long rows, int cols,
                               void* stream);

/* INT8 KV-cache append: quantizes n_new tokens per (b,h) of k_new/v_new
 * [BH, n_new, head_dim] (fp16, bf16 or fp32) per token into rows
 * pos .. pos+n_new-1 of K_cache/V_cache [BH, capacity, head_dim] and their
 * scales sK_cache/sV_cache [BH*capacity].  The producer side of decode; no
 * counterpart in the reference (its callers quantize the whole cache in
 * PyTorch, validation/check_decode.py:42-47). */
int int8k_kv_cache_append(const void* k_new, const void* v_new, int dtype,
                          int8_t* K_cache, int8_t* V_cache, float* sK_cache, float* sV_cache,
                          int BH, int n_new, int pos, int capacity, int head_dim, void* stream);

/* ------------------------------------------------------------------------ */
/* Producer-fused quantizers (quantize on emit).  The reference quantizes    */
/* every INT8 kernel input in a separate eager pass after its fp16 producer  */
/* (bench/bench_block.py:59-63, 104-110, 119-121, 138-139); these do the     */
/* producer and the quantization in one pass.  No reference counterpart.    */
/* ------------------------------------------------------------------------ */

/* LayerNorm over the last dim, then per-token int8 (the MLP input):
 *   y = (x - mean) / sqrt(var + eps) [* gamma] [+ beta]  (fp32, biased var),
 *   rounded to x's dtype (as F.layer_norm returns it), then
 *   scales[r] = max(amax_r(y), 1e-8) / 127, q = rn(clamp(y / s, -128, 127)).
 * x [rows, cols] of `dtype` (int8k_dtype); gamma/beta fp32 [cols] or NULL;
 * q int8 [rows, cols]; scales fp32 [rows]; y_out [rows, cols] of `dtype`
 * receives y when non-NULL. */
int int8k_layernorm_quantize_per_token(const void* x, int dtype, const float* gamma,
                                       const float* beta, float eps, int8_t* q, float* scales,
                                       void* y_out, long long rows, int cols, void* stream);

/* Splits a projection output x [B, S, parts, H, head_dim] (parts = 3 for a
 * fused QKV projection) into heads and quantizes each head row per token:
 * part p goes to q_p int8 [B, H, S, head_dim] and s_p fp32 [B, H, S] — the
 * inputs of int8k_attention_forward / the decode calls.  Pointers of parts
 * >= `parts` are ignored. */
int int8k_quantize_heads(const void* x, int dtype, int parts, int8_t* q0, float* s0,
                         int8_t* q1, float* s1, int8_t* q2, float* s2, int B, int S, int H,
                         int head_dim, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INT8K_H */
