/*
 * oracle_c.c — C restatement of the reference's CPU math — TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (as a second, independent implementation next to the numpy
 * oracle in int8_oracle.py) and by bench.py's cpu_baseline leg (the CPU
 * "port" the GPU numbers are reported beside).  The product library never
 * links or calls it.
 *
 *  oracle_decode_attention : dequant -> softmax attention for one query token
 *      per (b,h), float64, two-pass (max, then exp-sum) softmax.  Follows the
 *      contract of int8_decode_attention_forward
 *      (kernels/int8_decode_attention.cu:333, 361, 415-425, 448) as checked by
 *      validation/check_decode.py:65-68.
 *  oracle_prefill_attention : the same for seq_q == seq_kv, optional causal
 *      mask (kernels/int8_attention.cu:292-298, 467-643; causal is new).
 *  oracle_gemm_i8_i32 : exact s8 x s8 -> s32 product (kernels/int8_mlp.cu:242-310),
 *      int64 accumulation, returns 1 if any sum leaves the int32 range.
 *
 * Parallelised over independent rows with OpenMP; `threads` <= 0 keeps the
 * OpenMP default.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static void set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Q [BH,D] int8, K/V [BH,S,D] int8, sQ [BH], sK/sV [BH*S]; out [BH,D] float64. */
int oracle_decode_attention(const int8_t* Q, const int8_t* K, const int8_t* V,
                            const float* sQ, const float* sK, const float* sV,
                            long long BH, long long S, int D, double* out, int threads) {
    if (BH <= 0 || S <= 0 || D <= 0) return 1;
    set_threads(threads);
    const double scale = 1.0 / sqrt((double)D);
    int err = 0;
#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * (size_t)S);
        double* acc = (double*)malloc(sizeof(double) * (size_t)D);
        if (!sc || !acc) {
#pragma omp atomic write
            err = 1;
        }
#pragma omp for schedule(static)
        for (long long bh = 0; bh < BH; ++bh) {
            if (!sc || !acc) continue;
            const int8_t* q = Q + bh * D;
            const int8_t* k = K + bh * S * D;
            const int8_t* v = V + bh * S * D;
            const double qs = (double)sQ[bh] * scale;
            double mx = -INFINITY;
            for (long long j = 0; j < S; ++j) {
                long long dot = 0;
                const int8_t* kj = k + j * D;
                for (int d = 0; d < D; ++d) dot += (long long)q[d] * (long long)kj[d];
                sc[j] = (double)dot * qs * (double)sK[bh * S + j];
                if (sc[j] > mx) mx = sc[j];
            }
            double l = 0.0;
            for (int d = 0; d < D; ++d) acc[d] = 0.0;
            for (long long j = 0; j < S; ++j) {
                const double p = exp(sc[j] - mx);
                l += p;
                const double w = p * (double)sV[bh * S + j];
                const int8_t* vj = v + j * D;
                for (int d = 0; d < D; ++d) acc[d] += w * (double)vj[d];
            }
            for (int d = 0; d < D; ++d) out[bh * D + d] = acc[d] / l;
        }
        free(sc);
        free(acc);
    }
    return err;
}

/* Q/K/V [BH,S,D] int8, scales [BH*S]; out [BH,S,D] float64. */
int oracle_prefill_attention(const int8_t* Q, const int8_t* K, const int8_t* V,
                             const float* sQ, const float* sK, const float* sV,
                             long long BH, long long S, int D, int causal, double* out,
                             int threads) {
    if (BH <= 0 || S <= 0 || D <= 0) return 1;
    set_threads(threads);
    const double scale = 1.0 / sqrt((double)D);
    int err = 0;
#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * (size_t)S);
        double* acc = (double*)malloc(sizeof(double) * (size_t)D);
        if (!sc || !acc) {
#pragma omp atomic write
            err = 1;
        }
#pragma omp for schedule(dynamic, 16) collapse(2)
        for (long long bh = 0; bh < BH; ++bh) {
            for (long long i = 0; i < S; ++i) {
                if (!sc || !acc) continue;
                const int8_t* q = Q + (bh * S + i) * D;
                const double qs = (double)sQ[bh * S + i] * scale;
                const long long jn = causal ? i + 1 : S;
                double mx = -INFINITY;
                for (long long j = 0; j < jn; ++j) {
                    const int8_t* kj = K + (bh * S + j) * D;
                    long long dot = 0;
                    for (int d = 0; d < D; ++d) dot += (long long)q[d] * (long long)kj[d];
                    sc[j] = (double)dot * qs * (double)sK[bh * S + j];
                    if (sc[j] > mx) mx = sc[j];
                }
                double l = 0.0;
                for (int d = 0; d < D; ++d) acc[d] = 0.0;
                for (long long j = 0; j < jn; ++j) {
                    const double p = exp(sc[j] - mx);
                    l += p;
                    const double w = p * (double)sV[bh * S + j];
                    const int8_t* vj = V + (bh * S + j) * D;
                    for (int d = 0; d < D; ++d) acc[d] += w * (double)vj[d];
                }
                for (int d = 0; d < D; ++d) out[(bh * S + i) * D + d] = acc[d] / l;
            }
        }
        free(sc);
        free(acc);
    }
    return err;
}

/* C[M,N] = A[M,K] @ B[K,N], all row-major. Returns 1 on int32 overflow. */
int oracle_gemm_i8_i32(const int8_t* A, const int8_t* B, int32_t* C, long long M, long long N,
                       long long K, int threads) {
    set_threads(threads);
    int overflow = 0;
#pragma omp parallel
    {
        int64_t* row = (int64_t*)malloc(sizeof(int64_t) * (size_t)(N > 0 ? N : 1));
#pragma omp for schedule(static)
        for (long long m = 0; m < M; ++m) {
            if (!row) continue;
            memset(row, 0, sizeof(int64_t) * (size_t)N);
            const int8_t* a = A + m * K;
            for (long long k = 0; k < K; ++k) {
                const int64_t av = a[k];
                if (av == 0) continue;
                const int8_t* b = B + k * N;
                for (long long n = 0; n < N; ++n) row[n] += av * (int64_t)b[n];
            }
            for (long long n = 0; n < N; ++n) {
                if (row[n] > INT32_MAX || row[n] < INT32_MIN) {
#pragma omp atomic write
                    overflow = 1;
                }
                C[m * N + n] = (int32_t)row[n];
            }
        }
        free(row);
    }
    return overflow;
}
