// C-ABI shim over the reference's own CPU code -- TEST INFRASTRUCTURE ONLY.
//
// oracle/Makefile compiles this file together with the reference's
// src/backend/backend_naive.cc and src/quantize/quantize.cc, read in place
// from the reference tree (nothing is copied), into oracle/_ref/.  The
// result is the reference's BackendCPU operators (linear_q8 / linear_q8_add
// and the other ops of a decode step) and quantize_per_channel, callable
// through ctypes, used to check the oracle's restatement bit-for-bit and to
// write the golden vectors.
#include <cstddef>
#include <cstdint>
#include <cstring>

#include "src/backend/backend_naive.h"
#include "vvllm/quantize/quantize.h"

extern "C" {

void ref_quantize_per_channel(const float* weight, std::size_t N, std::size_t K, int8_t* q,
                              float* scales)
{
    vvllm::QuantizedWeight qw = vvllm::quantize_per_channel(weight, N, K);
    std::memcpy(q, qw.data.data(), N * K);
    std::memcpy(scales, qw.scales.data(), N * sizeof(float));
}

void ref_linear_q8(float* out, const float* inp, const int8_t* weight, const float* scales,
                   const float* bias, std::size_t M, std::size_t N, std::size_t K)
{
    vvllm::BackendCPU backend;
    backend.linear_q8(out, inp, weight, scales, bias, M, N, K);
}

void ref_linear_q8_add(float* out, const float* inp, const int8_t* weight, const float* scales,
                       const float* bias, const float* residual, std::size_t M, std::size_t N,
                       std::size_t K)
{
    vvllm::BackendCPU backend;
    backend.linear_q8_add(out, inp, weight, scales, bias, residual, M, N, K);
}

// The other BackendCPU operators, as the reference computes them.
void ref_add(float* out, const float* x, const float* y, std::size_t n) { vvllm::BackendCPU().add(out, x, y, n); }
void ref_mul(float* out, const float* x, const float* y, std::size_t n) { vvllm::BackendCPU().mul(out, x, y, n); }
void ref_silu(float* out, const float* x, std::size_t n) { vvllm::BackendCPU().silu(out, x, n); }
void ref_silu_mul(float* out, const float* gate, const float* up, std::size_t n)
{
    vvllm::BackendCPU().silu_mul(out, gate, up, n);
}
void ref_rms_norm(float* out, const float* x, const float* w, std::size_t n, float eps)
{
    vvllm::BackendCPU().rms_norm(out, x, w, n, eps);
}
void ref_softmax(float* out, const float* x, std::size_t n) { vvllm::BackendCPU().softmax(out, x, n); }
void ref_rope(float* q, float* k, std::size_t seq_len, std::size_t num_heads, std::size_t num_kv_heads,
              std::size_t head_dim, std::size_t pos, float theta)
{
    vvllm::BackendCPU().rope(q, k, seq_len, num_heads, num_kv_heads, head_dim, pos, theta);
}
void ref_linear(float* out, const float* inp, const float* w, const float* bias, std::size_t M, std::size_t N,
                std::size_t K)
{
    vvllm::BackendCPU().linear(out, inp, w, bias, M, N, K);
}
void ref_linear_add(float* out, const float* inp, const float* w, const float* bias, const float* residual,
                    std::size_t M, std::size_t N, std::size_t K)
{
    vvllm::BackendCPU().linear_add(out, inp, w, bias, residual, M, N, K);
}
void ref_matmul(float* out, const float* A, const float* B, std::size_t M, std::size_t N, std::size_t K)
{
    vvllm::BackendCPU().matmul(out, A, B, M, N, K);
}
void ref_causal_attention(float* out, const float* q, std::size_t q_idx, const float* k, const float* v,
                          std::size_t attend_len, std::size_t num_heads, std::size_t num_kv_heads,
                          std::size_t head_dim, float scale)
{
    vvllm::BackendCPU().causal_attention(out, q, q_idx, k, v, attend_len, num_heads, num_kv_heads, head_dim, scale);
}

}  // extern "C"
