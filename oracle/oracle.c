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

/* ---- the other BackendCPU operators (src/backend/backend_naive.cc) ---- */

/* :44-50, :52-58 */
void orc_add(float* out, const float* x, const float* y, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = x[i] + y[i];
}
void orc_mul(float* out, const float* x, const float* y, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = x[i] * y[i];
}

/* :60-66: x * (1 / (1 + exp(-x))) */
void orc_silu(float* out, const float* x, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = x[i] * (1 / (1.0f + expf(-x[i])));
}

/* :293-300: (v / (1 + exp(-v))) * up */
void orc_silu_mul(float* out, const float* gate, const float* up, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        float v = gate[i];
        out[i] = (v / (1.0f + expf(-v))) * up[i];
    }
}

/* :68-76: sequential sum of squares (std::accumulate), sqrt(sum / n + eps),
 * x / rms * w */
void orc_rms_norm(float* out, const float* x, const float* weight, size_t n, float eps)
{
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) sum = sum + x[i] * x[i];
    float rms = sqrtf(sum / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] / rms * weight[i];
}

/* :78-91 */
void orc_softmax(float* out, const float* x, size_t n)
{
    float max_val = x[0];
    for (size_t i = 1; i < n; i++)
        if (max_val < x[i]) max_val = x[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        out[i] = expf(x[i] - max_val);
        sum += out[i];
    }
    for (size_t i = 0; i < n; i++) out[i] /= sum;
}

/* :93-137: split-half pairs (i, i + half) of every q and k head */
static void rope_heads(float* base, size_t heads, size_t head_dim, size_t position, float theta)
{
    size_t half = head_dim / 2;
    for (size_t h = 0; h < heads; h++) {
        float* head = base + h * head_dim;
        for (size_t i = 0; i < half; i++) {
            float freq = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
            float angle = (float)position * freq;
            float cos_a = cosf(angle);
            float sin_a = sinf(angle);
            float x0 = head[i];
            float x1 = head[i + half];
            head[i] = x0 * cos_a - x1 * sin_a;
            head[i + half] = x0 * sin_a + x1 * cos_a;
        }
    }
}
void orc_rope(float* q, float* k, size_t seq_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
              size_t pos, float theta)
{
    for (size_t s = 0; s < seq_len; s++) {
        rope_heads(q + s * num_heads * head_dim, num_heads, head_dim, pos + s, theta);
        rope_heads(k + s * num_kv_heads * head_dim, num_kv_heads, head_dim, pos + s, theta);
    }
}

/* :139-156: sum starts at the bias, k in order */
void orc_linear(float* out, const float* inp, const float* weight, const float* bias, size_t M, size_t N, size_t K)
{
    for (size_t i = 0; i < M; i++)
        for (size_t j = 0; j < N; j++) {
            float sum = bias ? bias[j] : 0.0f;
            for (size_t k = 0; k < K; k++) sum += inp[i * K + k] * weight[j * K + k];
            out[i * N + j] = sum;
        }
}

/* :302-320: sum starts at the residual, then the bias, k in order */
void orc_linear_add(float* out, const float* inp, const float* weight, const float* bias, const float* residual,
                    size_t M, size_t N, size_t K)
{
    for (size_t i = 0; i < M; i++)
        for (size_t j = 0; j < N; j++) {
            float sum = residual[i * N + j];
            if (bias) sum += bias[j];
            for (size_t k = 0; k < K; k++) sum += inp[i * K + k] * weight[j * K + k];
            out[i * N + j] = sum;
        }
}

/* :25-42 */
void orc_matmul(float* out, const float* A, const float* B, size_t M, size_t N, size_t K)
{
    for (size_t i = 0; i < M; i++)
        for (size_t j = 0; j < N; j++) {
            float sum = 0.0f;
            for (size_t k = 0; k < K; k++) sum += A[i * K + k] * B[k * N + j];
            out[i * N + j] = sum;
        }
}

/* :344-378: per head, scores = (q . k) * scale, softmax, then
 * out[d] += p_t * v_t[d] in t order */
void orc_causal_attention(float* out, const float* q, size_t q_idx, const float* k, const float* v, size_t attend_len,
                          size_t num_heads, size_t num_kv_heads, size_t head_dim, float scale)
{
    size_t groups = num_heads / num_kv_heads;
    float* scores = (float*)malloc(attend_len * sizeof(float) + 4);
    for (size_t h = 0; h < num_heads; h++) {
        size_t kv_h = h / groups;
        const float* q_head = q + q_idx * num_heads * head_dim + h * head_dim;
        for (size_t t = 0; t < attend_len; t++) {
            const float* k_head = k + t * num_kv_heads * head_dim + kv_h * head_dim;
            float dot = 0.0f;
            for (size_t d = 0; d < head_dim; d++) dot += q_head[d] * k_head[d];
            scores[t] = dot * scale;
        }
        orc_softmax(scores, scores, attend_len);
        float* head_out = out + h * head_dim;
        memset(head_out, 0, head_dim * sizeof(float));
        for (size_t t = 0; t < attend_len; t++) {
            const float* v_head = v + t * num_kv_heads * head_dim + kv_h * head_dim;
            for (size_t d = 0; d < head_dim; d++) head_out[d] += scores[t] * v_head[d];
        }
    }
    free(scores);
}

/* ---- sampling ----------------------------------------------------------
 * SamplerCPU::sample's greedy branch (src/sampler/sampler.cc:21-25) and the
 * device sampler SamplerCUDA::sample -> cuda_sample
 * (src/sampler/sampler_cuda.cc:13-18, src/backend/cuda_kernels.cu:1228-1349). */

/* gpu_rand's hash (cuda_kernels.cu:1230-1235): the seed xor a Weyl step of
 * (step, idx), then the splitmix64 finaliser. */
uint64_t orc_sample_hash(uint64_t seed, int32_t step, int32_t idx)
{
    uint64_t h = seed ^ ((uint64_t)(int64_t)step * 0x9E3779B97F4A7C15ull + (uint64_t)(int64_t)idx * 0x517CC1B727220A95ull);
    h = (h ^ (h >> 30)) * 0xBF58476D1CE4E5B9ull;
    h = (h ^ (h >> 27)) * 0x94D049BB133111EBull;
    return h ^ (h >> 31);
}

/* gpu_rand (:1228-1237): the top 53 bits to fp32, times 2^-53, plus 1e-10. */
float orc_sample_uniform(uint64_t seed, int32_t step, int32_t idx)
{
    const uint64_t h = orc_sample_hash(seed, step, idx);
    return (float)(h >> 11) * (1.0f / (float)(1ULL << 53)) + 1e-10f;
}

/* temperature == 0: the first index of the maximum (std::max_element,
 * sampler.cc:21-25).  temperature > 0: sample_kernel's Gumbel-max branch
 * (:1287-1316) in index order: noisy_i = logit_i / T - log(-log(u_i)); a
 * candidate replaces the best only when strictly greater, from a start of
 * -1e30 at index 0.  best / second (optional) receive the two largest noisy
 * values, so a caller can tell a near-tie. */
int32_t orc_sample(const float* logits, size_t n, float temperature, uint64_t seed, int32_t step, float* best,
                   float* second)
{
    if (temperature == 0.0f) {
        size_t bi = 0;
        for (size_t i = 1; i < n; i++)
            if (logits[bi] < logits[i]) bi = i;
        if (best) *best = n ? logits[bi] : 0.0f;
        if (second) *second = -INFINITY;
        return (int32_t)bi;
    }
    float bv = -1e30f, sv = -INFINITY;
    int32_t bi = 0;
    for (size_t i = 0; i < n; i++) {
        const float u = orc_sample_uniform(seed, step, (int32_t)i);
        const float g = -logf(-logf(u));
        const float v = logits[i] / temperature + g;
        if (v > bv) {
            sv = bv;
            bv = v;
            bi = (int32_t)i;
        } else if (v > sv) {
            sv = v;
        }
    }
    if (best) *best = bv;
    if (second) *second = sv;
    return bi;
}
