// BackendHIP: the MI355X backend of the INT8 per-channel linear path.
//
// A drop-in for BackendCUDA (src/backend/backend_cuda.h:14-84):
// linear_q8 / linear_q8_add run hand-written gfx950 kernels through the C
// ABI of libvvllm_hip.so (include/vvllm_hip.h), and so do the other
// operators of a decode step (norm, RoPE, attention, SiLU-mul, embedding,
// dense linear, ...).  Weights, scales, biases, norm weights and tables are
// host pointers mirrored to HBM on first use; activations are device
// pointers (fp32, or fp16 when constructed with fp16 = true, like
// BackendCUDA(bool fp16), backend_cuda.cc:13-26).  KVCacheHIP keeps the
// per-layer K/V rows in HBM.
//
// Failures of the C ABI are raised as std::runtime_error carrying the
// library's message (the reference exits the process instead).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_set>
#include <vector>

#include "vvllm/backend/backend.h"
#include "vvllm/kv_cache/kv_cache.h"

namespace vvllm
{

class BackendHIP : public Backend
{
public:
    explicit BackendHIP(bool fp16 = false, int device = 0);
    ~BackendHIP() override;

    BackendHIP(const BackendHIP&) = delete;
    BackendHIP& operator=(const BackendHIP&) = delete;

    bool fp16() const { return fp16_; }
    const std::string& device_name() const { return name_; }

    // pinned host staging memory (BackendCUDA::allocate, backend_cuda.cc:40-41)
    void* allocate(std::size_t bytes) override;
    void deallocate(void* ptr) override;

    // ---- the int8 path ----
    void linear_q8(float* out, const float* inp, const int8_t* weight, const float* scales,
                   const float* bias, std::size_t M, std::size_t N, std::size_t K) override;
    void linear_q8_add(float* out, const float* inp, const int8_t* weight, const float* scales,
                       const float* bias, const float* residual, std::size_t M, std::size_t N,
                       std::size_t K) override;
    bool is_fp16() const override { return fp16_; }
    Device device() const override { return Device::HIP; }
    void fp32_to_fp16(void* dst, const float* src, std::size_t n) override;
    void fp16_to_fp32(float* dst, const void* src, std::size_t n) override;

    // Quantizes host weight rows (BF16 when bf16, else F32; N x K, e.g. an
    // mmap'ed safetensors tensor) straight into the HBM mirror and writes the
    // N scales to `scales`.  Returns the pointer to pass as `weight` (with
    // the same scales and bias pointers) to linear_q8 / linear_q8_add: the
    // call then finds this mirror, with codes bit-identical to
    // quantize_per_channel of the widened rows.  Replaces, for this backend,
    // the host widening and quantization of Qwen2Model::load_weights
    // (src/model/qwen2/model.cc:27-33).
    const int8_t* ingest_weight(const void* host_rows, bool bf16, const float* bias, std::size_t N,
                                std::size_t K, float* scales);

    // Drops the HBM mirror of a host weight (e.g. before its buffer is freed
    // and reused); the next linear_q8 on that pointer uploads again.
    void forget_weight(const int8_t* host_weight);

    // ---- the other operators of a decode step ----
    void matmul(float*, const float*, const float*, std::size_t, std::size_t, std::size_t) override;
    void add(float*, const float*, const float*, std::size_t) override;
    void mul(float*, const float*, const float*, std::size_t) override;
    void silu(float*, const float*, std::size_t) override;
    void rms_norm(float*, const float*, const float*, std::size_t, float) override;
    void softmax(float*, const float*, std::size_t) override;
    void rope(float*, float*, std::size_t, std::size_t, std::size_t, std::size_t, std::size_t,
              float) override;
    void linear(float*, const float*, const float*, const float*, std::size_t, std::size_t,
                std::size_t) override;
    void silu_mul(float*, const float*, const float*, std::size_t) override;
    void linear_add(float*, const float*, const float*, const float*, const float*, std::size_t,
                    std::size_t, std::size_t) override;
    void embedding(float*, const float*, std::size_t, std::size_t, std::size_t) override;
    void causal_attention(float*, const float*, std::size_t, const float*, const float*,
                          std::size_t, std::size_t, std::size_t, std::size_t, float) override;

private:
    std::uint64_t mirror(const int8_t* weight, const float* scales, const float* bias,
                         std::size_t N, std::size_t K);
    int act_dtype() const;
    std::size_t elem() const;
    const void* host_mirror(const float* host, std::size_t n, int as_dtype);

    bool fp16_;
    std::string name_;
    // Mirrors this backend created or used, released by the destructor, as
    // BackendCUDA frees its per-instance weight caches (backend_cuda.cc:28-35):
    // a later backend never sees device copies keyed by host addresses that
    // may since have been freed and reused.
    std::unordered_set<std::uint64_t> weights_;
    std::unordered_set<const float*> arrays_;
};

// Key/value cache in HBM (KVCacheCUDA, src/kv_cache/kv_cache_cuda.cc:22-95):
// per layer, rows of kv_dim values in the backend's activation dtype.
// append() queues one kernel on the null stream that copies the k and v
// rows (they come from device tensors).  reserve() sizes every layer for a whole context up
// front (one allocation per layer; 288 GB of HBM holds long contexts), so
// appends never reallocate.
class KVCacheHIP : public KVCache
{
public:
    explicit KVCacheHIP(bool fp16 = false);
    ~KVCacheHIP() override;
    KVCacheHIP(const KVCacheHIP&) = delete;
    KVCacheHIP& operator=(const KVCacheHIP&) = delete;

    void init(std::size_t num_layers, std::size_t kv_dim) override;
    void append(std::size_t layer, const float* k, const float* v, std::size_t num_tokens) override;
    const float* k(std::size_t layer) const override;
    const float* v(std::size_t layer) const override;
    void reset() override { seq_len_ = 0; }
    void truncate(std::size_t new_seq_len) override;

    void reserve(std::size_t tokens);
    std::size_t seq_len() const { return seq_len_; }

private:
    struct Layer {
        void* k = nullptr;
        void* v = nullptr;
        std::size_t cap = 0;  // tokens
    };
    void grow(Layer& l, std::size_t tokens);
    std::size_t elem() const { return fp16_ ? 2 : 4; }

    bool fp16_;
    std::size_t reserve_tokens_ = 128;
    std::vector<Layer> layers_;
};

// Tensor-layer hooks for Device::HIP: the bodies of device_allocate /
// device_deallocate / device_copy (src/tensor/tensor.cc:72-116) for the GPU
// device, backed by the caching allocator of libvvllm_hip.
void* hip_device_allocate(std::size_t bytes);
void hip_device_deallocate(void* ptr);
void hip_copy_h2d(void* dst, const void* src, std::size_t bytes);
void hip_copy_d2h(void* dst, const void* src, std::size_t bytes);
void hip_copy_d2d(void* dst, const void* src, std::size_t bytes);

}  // namespace vvllm
