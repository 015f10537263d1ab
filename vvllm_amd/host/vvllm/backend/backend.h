// The vvllm operator interface a backend implements.
//
// Method names, parameter lists and their meaning are the reference's
// (include/vvllm/backend/backend.h:18-114) so that model code written against
// it (transformer_forward, the IR executable) calls a BackendHIP unchanged.
// All pointers are raw: host pointers for weights, scales and biases; for
// activations, device pointers when device() is a GPU.  When is_fp16() is
// true, activation/output buffers hold half values behind the float*.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>

#include "vvllm/tensor/device.h"

namespace vvllm
{

enum class BackendKind
{
    CPU,
    BLAS,
};

class Backend
{
public:
    virtual ~Backend() = default;

    // memory (host staging buffers)
    virtual void* allocate(std::size_t bytes) = 0;
    virtual void deallocate(void* ptr) = 0;

    // out[M,N] = A[M,K] * B[K,N]
    virtual void matmul(float* out, const float* A, const float* B, std::size_t M, std::size_t N,
                        std::size_t K) = 0;
    // element-wise
    virtual void add(float* out, const float* x, const float* y, std::size_t n) = 0;
    virtual void mul(float* out, const float* x, const float* y, std::size_t n) = 0;
    virtual void silu(float* out, const float* x, std::size_t n) = 0;
    // out = x / sqrt(mean(x^2) + eps) * weight
    virtual void rms_norm(float* out, const float* x, const float* weight, std::size_t n,
                          float eps) = 0;
    virtual void softmax(float* out, const float* x, std::size_t n) = 0;
    // in-place rotary embedding of q[seq, heads, hd] and k[seq, kv_heads, hd]
    virtual void rope(float* q, float* k, std::size_t seq_len, std::size_t num_heads,
                      std::size_t num_kv_heads, std::size_t head_dim, std::size_t pos,
                      float theta) = 0;
    // out[M,N] = inp[M,K] . weight[N,K]^T + bias[N]; bias may be null
    virtual void linear(float* out, const float* inp, const float* weight, const float* bias,
                        std::size_t M, std::size_t N, std::size_t K) = 0;
    // out[M,N] = (inp[M,K] . q[N,K]^T) * scales[N] + bias[N]; q int8 row-major; bias may be null
    virtual void linear_q8(float* out, const float* inp, const int8_t* weight, const float* scales,
                           const float* bias, std::size_t M, std::size_t N, std::size_t K) = 0;
    // out = silu(gate) * up
    virtual void silu_mul(float* out, const float* gate, const float* up, std::size_t n) = 0;
    // linear + residual; out may alias residual
    virtual void linear_add(float* out, const float* inp, const float* weight, const float* bias,
                            const float* residual, std::size_t M, std::size_t N,
                            std::size_t K) = 0;
    // linear_q8 + residual; out may alias residual
    virtual void linear_q8_add(float* out, const float* inp, const int8_t* weight,
                               const float* scales, const float* bias, const float* residual,
                               std::size_t M, std::size_t N, std::size_t K) = 0;
    // out[hidden] = table[token_id * hidden ...]
    virtual void embedding(float* out, const float* table, std::size_t token_id,
                           std::size_t hidden_size, std::size_t vocab_size) = 0;
    // causal multi-head attention of one query position against attend_len keys
    virtual void causal_attention(float* out, const float* q, std::size_t q_idx, const float* k,
                                  const float* v, std::size_t attend_len, std::size_t num_heads,
                                  std::size_t num_kv_heads, std::size_t head_dim, float scale) = 0;

    // optional hooks (no-ops unless a backend needs them)
    virtual void begin_forward() {}
    virtual void flush(const void* /*ptr*/, std::size_t /*bytes*/) {}
    virtual const void* device_ptr(const void* /*host_ptr*/) const { return nullptr; }
    virtual bool is_fp16() const { return false; }
    virtual void fp32_to_fp16(void* /*dst*/, const float* /*src*/, std::size_t /*n*/) {}
    virtual void fp16_to_fp32(float* /*dst*/, const void* /*src*/, std::size_t /*n*/) {}
    virtual Device device() const { return Device::CPU; }
};

std::unique_ptr<Backend> create_backend(BackendKind kind);

}  // namespace vvllm
