/*
 * CPU oracle for the INT8 per-channel linear path -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker, never the product: only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it.  The product path (libvvllm_hip.so / BackendHIP) never calls it and has
 * no CPU fallback.
 *
 * Every function restates one reference routine (file:line relative to the
 * vvllm source tree) operation for operation, so that its results can be
 * compared bit-for-bit with the reference compiled from its own sources
 * (oracle/_ref, see oracle/Makefile) and with the committed golden vectors.
 *
 * Pinning status (see tests/test_oracle.py):
 *   orc_quantize_per_channel  pinned: reference KATs (quantize_test.cc),
 *                             closed-form tie/NaN/Inf cases, bit-exact vs _ref
 *   orc_linear_q8             pinned: reference KATs (backend_naive_test.cc),
 *                             exact-integer closed forms, fp64 brute force,
 *                             bit-exact vs _ref and the golden vectors
 *   orc_linear_q8_add         pinned: bit-exact vs _ref and golden vectors,
 *                             identity with orc_linear_q8 + fp32 add
 *   orc_linear_q8_f64         pinned: exact on integer-valued inputs (closed
 *                             form), agreement with orc_linear_q8 within the
 *                             fp32 error bound
 *   orc_bf16_to_f32           pinned: the closed-form BF16 decoding
 *                             (-1)^s 2^(e-127) (1 + m/128), subnormals, +-0,
 *                             +-Inf and NaN, for all 65536 bit patterns
 *   orc_ingest_bf16           composition of the two above (the host path
 *                             vvh_weight_ingest replaces); pinned through them
 *   orc_add/mul/silu/silu_mul, orc_rms_norm, orc_softmax, orc_rope,
 *   orc_linear, orc_linear_add, orc_matmul, orc_causal_attention
 *                             pinned: bit-exact vs the reference's BackendCPU
 *                             compiled in place (_ref), plus closed forms
 *                             (tests/test_oracle.py)
 *   orc_sample_hash           pinned: splitmix64's published outputs for seed
 *                             0 (the step term is its Weyl sequence), bit
 *                             mixing of the index term (avalanche)
 *   orc_sample_uniform        pinned: closed form of the top-53-bit scaling,
 *                             uniformity (Kolmogorov-Smirnov) over indices
 *   orc_sample                pinned: temperature 0 = std::max_element,
 *                             one-hot and dominant logits, chi-square of the
 *                             sampled frequencies against softmax(logit / T),
 *                             and a planted sign error in the Gumbel term
 *                             rejected by the same test
 */
#ifndef VVLLM_ORACLE_H
#define VVLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SafeTensorsLoader::bf16_to_f32, src/safetensors/safetensors.cc:135-141,
 * applied elementwise as load_tensor does for BF16 tensors (:112-119). */
void orc_bf16_to_f32(const uint16_t* src, size_t n, float* dst);

/* The host path of a BF16 weight: widen (above), then quantize_per_channel
 * (src/model/qwen2/model.cc:27-33 on a tensor from load_tensor). */
void orc_ingest_bf16(const uint16_t* src, size_t N, size_t K, int8_t* q, float* scales);

/* quantize_per_channel, src/quantize/quantize.cc:9-48.
 * q: [N*K] int8 codes, scales: [N]. */
void orc_quantize_per_channel(const float* weight, size_t N, size_t K, int8_t* q, float* scales);

/* BackendCPU::linear_q8, src/backend/backend_naive.cc:155-291 (x86 AVX2+FMA
 * branch :216-274 and epilogue :283-288, the branch selected by the -mavx2
 * -mfma copts of src/backend/BUILD.bazel:5-8).  bias may be NULL. */
void orc_linear_q8(float* out, const float* inp, const int8_t* weight, const float* scales,
                   const float* bias, size_t M, size_t N, size_t K);

/* BackendCPU::linear_q8_add, src/backend/backend_naive.cc:322-335:
 * linear_q8 into out, then out = out + residual (two fp32 roundings);
 * out == residual is allowed (the residual is snapshotted first). */
void orc_linear_q8_add(float* out, const float* inp, const int8_t* weight, const float* scales,
                       const float* bias, const float* residual, size_t M, size_t N, size_t K);

/* Same contract as orc_linear_q8_add (residual may be NULL) evaluated in
 * double precision: out = scale*sum(x*q) + bias + residual.  Used for the
 * error-bound checks, not for parity. */
void orc_linear_q8_f64(double* out, const float* inp, const int8_t* weight, const float* scales,
                       const float* bias, const float* residual, size_t M, size_t N, size_t K);

/* Number of threads the oracle uses: always 1 (the reference is
 * single-threaded, README.md:282). */
int orc_threads(void);

/* The other BackendCPU operators, src/backend/backend_naive.cc (line ranges
 * in oracle.c). */
void orc_add(float* out, const float* x, const float* y, size_t n);
void orc_mul(float* out, const float* x, const float* y, size_t n);
void orc_silu(float* out, const float* x, size_t n);
void orc_silu_mul(float* out, const float* gate, const float* up, size_t n);
void orc_rms_norm(float* out, const float* x, const float* weight, size_t n, float eps);
void orc_softmax(float* out, const float* x, size_t n);
void orc_rope(float* q, float* k, size_t seq_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
              size_t pos, float theta);
void orc_linear(float* out, const float* inp, const float* weight, const float* bias, size_t M, size_t N, size_t K);
void orc_linear_add(float* out, const float* inp, const float* weight, const float* bias, const float* residual,
                    size_t M, size_t N, size_t K);
void orc_matmul(float* out, const float* A, const float* B, size_t M, size_t N, size_t K);
void orc_causal_attention(float* out, const float* q, size_t q_idx, const float* k, const float* v, size_t attend_len,
                          size_t num_heads, size_t num_kv_heads, size_t head_dim, float scale);

/* Sampling: SamplerCPU's greedy branch (src/sampler/sampler.cc:21-25) at
 * temperature 0 and the device sampler's Gumbel-max trick above it
 * (src/backend/cuda_kernels.cu:1228-1317; cuda_sample :1322-1349). */
uint64_t orc_sample_hash(uint64_t seed, int32_t step, int32_t idx);
float orc_sample_uniform(uint64_t seed, int32_t step, int32_t idx);
int32_t orc_sample(const float* logits, size_t n, float temperature, uint64_t seed, int32_t step, float* best,
                   float* second);

#ifdef __cplusplus
}
#endif

#endif
