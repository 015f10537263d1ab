/*
 * CPU oracle for the INT8 per-channel linear path -- TEST INFRASTRUCTURE ONLY.
 * (Checker for tests/, smoke() and bench.py's cpu_baseline; never linked into
 * the product.)  Restates the reference operation for operation; see oracle.h
 * for the per-function pinning status.
 *
 * Build: gcc -O2 -mavx2 -mfma (oracle/Makefile), the same ISA flags the
 * reference's CPU backend is compiled with (src/backend/BUILD.bazel:5-8).
 * The scalar tail keeps `sum += x*w` contractible (gcc's default
 * -ffp-contract=fast for GNU C), as the reference's C++ is.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* std::max(a, b) == (a < b) ? b : a ; std::min(a, b) == (b < a) ? b : a.
 * The argument order decides what happens to NaN (quantize.cc:21, :40). */
static inline float std_max(float a, float b) { return (a < b) ? b : a; }
static inline float std_min(float a, float b) { return (b < a) ? b : a; }

/* src/quantize/quantize.cc:9-48 */
void orc_quantize_per_channel(const float* weight, size_t N, size_t K, int8_t* q, float* scales)
{
    for (size_t j = 0; j < N; j++) {
        const float* row = weight + j * K;
        float absmax = 0.0f;                         /* :18-22 */
        for (size_t k = 0; k < K; k++) absmax = std_max(absmax, fabsf(row[k]));
        float scale = absmax / 127.0f;               /* :24 */
        scales[j] = scale;                           /* :25 */
        if (scale == 0.0f) {                         /* :27-34 */
            memset(q + j * K, 0, K);
            continue;
        }
        float inv_scale = 1.0f / scale;              /* :37 */
        for (size_t k = 0; k < K; k++) {             /* :38-43 */
            float val = row[k] * inv_scale;
            val = std_max(-128.0f, std_min(127.0f, roundf(val)));
            q[j * K + k] = (int8_t)val;
        }
    }
}

/* src/safetensors/safetensors.cc:135-141: the BF16 bits become the high half
 * of the fp32 word (exact). */
void orc_bf16_to_f32(const uint16_t* src, size_t n, float* dst)
{
    for (size_t i = 0; i < n; i++) {
        uint32_t bits = (uint32_t)src[i] << 16;
        memcpy(&dst[i], &bits, sizeof(float));
    }
}

/* load_tensor's BF16 branch (safetensors.cc:112-119) then quantize_per_channel
 * (src/model/qwen2/model.cc:27-33). */
void orc_ingest_bf16(const uint16_t* src, size_t N, size_t K, int8_t* q, float* scales)
{
    float* w = (float*)malloc(N * K * sizeof(float) + 1);
    orc_bf16_to_f32(src, N * K, w);
    orc_quantize_per_channel(w, N, K, q, scales);
    free(w);
}

/* One output element of BackendCPU::linear_q8, AVX2+FMA branch,
 * src/backend/backend_naive.cc:216-274. */
static float dot_avx2(const float* in_row, const int8_t* w_row, size_t K)
{
    __m256 acc0 = _mm256_setzero_ps();
    __m256 acc1 = _mm256_setzero_ps();
    __m256 acc2 = _mm256_setzero_ps();
    __m256 acc3 = _mm256_setzero_ps();
    size_t k = 0;
    for (; k + 32 <= K; k += 32) {                                        /* :228 */
        __m256i w8 = _mm256_loadu_si256((const __m256i*)(w_row + k));
        __m128i lo16 = _mm256_castsi256_si128(w8);
        __m128i hi16 = _mm256_extracti128_si256(w8, 1);
        /* bytes 0-7, 8-15, 16-23, 24-31 -> int32 -> fp32 (exact) */
        __m256 w0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(lo16));
        __m256 w1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(lo16, 8)));
        __m256 w2 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(hi16));
        __m256 w3 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(hi16, 8)));
        acc0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(in_row + k), acc0);   /* :251-255 */
        acc1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(in_row + k + 8), acc1);
        acc2 = _mm256_fmadd_ps(w2, _mm256_loadu_ps(in_row + k + 16), acc2);
        acc3 = _mm256_fmadd_ps(w3, _mm256_loadu_ps(in_row + k + 24), acc3);
    }
    /* :258-268: (a0+a1)+(a2+a3), fold halves, two horizontal adds */
    __m256 s = _mm256_add_ps(_mm256_add_ps(acc0, acc1), _mm256_add_ps(acc2, acc3));
    __m128 r = _mm_add_ps(_mm256_castps256_ps128(s), _mm256_extractf128_ps(s, 1));
    r = _mm_hadd_ps(r, r);
    r = _mm_hadd_ps(r, r);
    float sum = _mm_cvtss_f32(r);
    for (; k < K; k++) sum += in_row[k] * (float)w_row[k];              /* :271-274 */
    return sum;
}

/* src/backend/backend_naive.cc:155-291 (epilogue :283-288) */
void orc_linear_q8(float* out, const float* inp, const int8_t* weight, const float* scales,
                   const float* bias, size_t M, size_t N, size_t K)
{
    for (size_t i = 0; i < M; i++) {
        const float* in_row = inp + i * K;
        for (size_t j = 0; j < N; j++) {
            float sum = dot_avx2(in_row, weight + j * K, K);
            sum *= scales[j];
            if (bias) sum += bias[j];
            out[i * N + j] = sum;
        }
    }
}

/* src/backend/backend_naive.cc:322-335 */
void orc_linear_q8_add(float* out, const float* inp, const int8_t* weight, const float* scales,
                       const float* bias, const float* residual, size_t M, size_t N, size_t K)
{
    float* snapshot = NULL;
    if (out == residual) {                                                /* :327-332 */
        snapshot = (float*)malloc(M * N * sizeof(float));
        memcpy(snapshot, residual, M * N * sizeof(float));
        residual = snapshot;
    }
    orc_linear_q8(out, inp, weight, scales, bias, M, N, K);
    for (size_t i = 0; i < M * N; i++) out[i] = out[i] + residual[i];    /* add(), :41-47 */
    free(snapshot);
}

void orc_linear_q8_f64(double* out, const float* inp, const int8_t* weight, const float* scales,
                       const float* bias, const float* residual, size_t M, size_t N, size_t K)
{
    for (size_t i = 0; i < M; i++) {
        for (size_t j = 0; j < N; j++) {
            double acc = 0.0;
            for (size_t k = 0; k < K; k++) acc += (double)inp[i * K + k] * (double)weight[j * K + k];
            double v = acc * (double)scales[j];
            if (bias) v += (double)bias[j];
            if (residual) v += (double)residual[i * N + j];
            out[i * N + j] = v;
        }
    }
}

int orc_threads(void) { return 1; }
