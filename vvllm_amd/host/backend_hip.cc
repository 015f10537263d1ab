// BackendHIP implementation: C++20 host code over the C ABI of
// libvvllm_hip.so.  See backend_hip.h.
#include "backend_hip.h"

#include <algorithm>
#include <stdexcept>
#include <string>

#include "vvllm_hip.h"

namespace vvllm
{

namespace
{

void check(int status, const char* what)
{
    if (status != VVH_OK)
    {
        throw std::runtime_error(std::string("BackendHIP: ") + what + ": " +
                                 vvh_status_string(status) + ": " + vvh_last_error());
    }
}

}  // namespace

BackendHIP::BackendHIP(bool fp16, int device) : fp16_(fp16)
{
    char name[256] = {0};
    check(vvh_init(device, name, sizeof(name)), "init");
    name_ = name;
}

BackendHIP::~BackendHIP()
{
    // a mirror may already be gone (forget_weight, or another backend that
    // shared it): those calls fail harmlessly
    for (const std::uint64_t h : weights_) (void)vvh_weight_release(h);
    for (const float* p : arrays_) (void)vvh_mirror_release(p);
}

void* BackendHIP::allocate(std::size_t bytes)
{
    void* p = nullptr;
    check(vvh_malloc_host(&p, bytes), "allocate");
    return p;
}

void BackendHIP::deallocate(void* ptr) { check(vvh_free_host(ptr), "deallocate"); }

int BackendHIP::act_dtype() const { return fp16_ ? VVH_F16 : VVH_F32; }

std::uint64_t BackendHIP::mirror(const int8_t* weight, const float* scales, const float* bias,
                                 std::size_t N, std::size_t K)
{
    vvh_weight h = 0;
    check(vvh_weight_register(weight, scales, bias, N, K, &h), "weight mirror");
    weights_.insert(h);
    return h;
}

// Backend::linear_q8 (include/vvllm/backend/backend.h:62-65); replaces
// BackendCUDA::linear_q8 (src/backend/backend_cuda.cc:188-213).
void BackendHIP::linear_q8(float* out, const float* inp, const int8_t* weight, const float* scales,
                           const float* bias, std::size_t M, std::size_t N, std::size_t K)
{
    if (M == 0 || N == 0) return;
    const vvh_weight h = mirror(weight, scales, bias, N, K);
    check(vvh_linear_q8(out, inp, h, nullptr, M, N, K, act_dtype(), act_dtype(), nullptr),
          "linear_q8");
}

// Backend::linear_q8_add (backend.h:75-78); replaces BackendCUDA::linear_q8_add
// (backend_cuda.cc:246-275).  out == residual is handled inside the kernel
// (each output element reads its residual before writing), so no copy is made.
void BackendHIP::linear_q8_add(float* out, const float* inp, const int8_t* weight,
                               const float* scales, const float* bias, const float* residual,
                               std::size_t M, std::size_t N, std::size_t K)
{
    if (M == 0 || N == 0) return;
    const vvh_weight h = mirror(weight, scales, bias, N, K);
    check(vvh_linear_q8(out, inp, h, residual, M, N, K, act_dtype(), act_dtype(), nullptr),
          "linear_q8_add");
}

void BackendHIP::fp32_to_fp16(void* dst, const float* src, std::size_t n)
{
    check(vvh_convert(dst, VVH_F16, src, VVH_F32, n, nullptr), "fp32_to_fp16");
}

void BackendHIP::fp16_to_fp32(float* dst, const void* src, std::size_t n)
{
    check(vvh_convert(dst, VVH_F32, src, VVH_F16, n, nullptr), "fp16_to_fp32");
}

const int8_t* BackendHIP::ingest_weight(const void* host_rows, bool bf16, const float* bias, std::size_t N,
                                        std::size_t K, float* scales)
{
    vvh_weight h = 0;
    check(vvh_weight_ingest(host_rows, bf16 ? VVH_BF16 : VVH_F32, bias, N, K, scales, &h), "ingest_weight");
    weights_.insert(h);
    return static_cast<const int8_t*>(host_rows);
}

void BackendHIP::forget_weight(const int8_t* host_weight)
{
    vvh_weight h = 0;
    if (vvh_weight_find(host_weight, &h) == VVH_OK) check(vvh_weight_release(h), "forget_weight");
}

// ---- the other operators of a decode step (C ABI: vvh_eltwise & co.) ----
// Weights, norm weights, biases and tables are host fp32 pointers, mirrored
// on first use (vvh_mirror_f32); dense weights are mirrored as fp16 in fp16
// mode (as BackendCUDA::linear does, backend_cuda.cc:171-181).
const void* BackendHIP::host_mirror(const float* host, std::size_t n, int as_dtype)
{
    const void* dev = nullptr;
    check(vvh_mirror_f32(host, n, as_dtype, &dev), "mirror");
    arrays_.insert(host);
    return dev;
}

std::size_t BackendHIP::elem() const { return fp16_ ? 2 : 4; }

void BackendHIP::matmul(float* out, const float* A, const float* B, std::size_t M, std::size_t N, std::size_t K)
{
    const float* dB = static_cast<const float*>(host_mirror(B, K * N, VVH_F32));
    check(vvh_matmul(out, A, dB, M, N, K, act_dtype(), nullptr), "matmul");
}

void BackendHIP::add(float* out, const float* x, const float* y, std::size_t n)
{
    check(vvh_eltwise(VVH_OP_ADD, out, x, y, n, act_dtype(), nullptr), "add");
}

void BackendHIP::mul(float* out, const float* x, const float* y, std::size_t n)
{
    check(vvh_eltwise(VVH_OP_MUL, out, x, y, n, act_dtype(), nullptr), "mul");
}

void BackendHIP::silu(float* out, const float* x, std::size_t n)
{
    check(vvh_eltwise(VVH_OP_SILU, out, x, nullptr, n, act_dtype(), nullptr), "silu");
}

void BackendHIP::silu_mul(float* out, const float* gate, const float* up, std::size_t n)
{
    check(vvh_eltwise(VVH_OP_SILU_MUL, out, gate, up, n, act_dtype(), nullptr), "silu_mul");
}

void BackendHIP::rms_norm(float* out, const float* x, const float* weight, std::size_t n, float eps)
{
    const float* dw = static_cast<const float*>(host_mirror(weight, n, VVH_F32));
    check(vvh_rms_norm(out, x, dw, 1, n, eps, act_dtype(), nullptr), "rms_norm");
}

void BackendHIP::softmax(float* out, const float* x, std::size_t n)
{
    check(vvh_softmax(out, x, 1, n, act_dtype(), nullptr), "softmax");
}

void BackendHIP::rope(float* q, float* k, std::size_t seq_len, std::size_t num_heads, std::size_t num_kv_heads,
                      std::size_t head_dim, std::size_t pos, float theta)
{
    check(vvh_rope(q, k, seq_len, num_heads, num_kv_heads, head_dim, pos, theta, act_dtype(), nullptr), "rope");
}

void BackendHIP::linear(float* out, const float* inp, const float* weight, const float* bias, std::size_t M,
                        std::size_t N, std::size_t K)
{
    const int wd = act_dtype();
    const void* dw = host_mirror(weight, N * K, wd);
    const float* db = bias ? static_cast<const float*>(host_mirror(bias, N, VVH_F32)) : nullptr;
    check(vvh_dense(out, inp, dw, wd, db, nullptr, M, N, K, act_dtype(), nullptr), "linear");
}

void BackendHIP::linear_add(float* out, const float* inp, const float* weight, const float* bias,
                            const float* residual, std::size_t M, std::size_t N, std::size_t K)
{
    const int wd = act_dtype();
    const void* dw = host_mirror(weight, N * K, wd);
    const float* db = bias ? static_cast<const float*>(host_mirror(bias, N, VVH_F32)) : nullptr;
    check(vvh_dense(out, inp, dw, wd, db, residual, M, N, K, act_dtype(), nullptr), "linear_add");
}

// Always fp32 out: transformer_forward embeds into an fp32 tensor and converts
// it itself in fp16 mode (include/vvllm/model/transformer.h:93-108).
void BackendHIP::embedding(float* out, const float* table, std::size_t token_id, std::size_t hidden_size,
                           std::size_t vocab_size)
{
    const float* dt = static_cast<const float*>(host_mirror(table, vocab_size * hidden_size, VVH_F32));
    check(vvh_embedding(out, dt, token_id, hidden_size, vocab_size, VVH_F32, nullptr), "embedding");
}

// q is the whole [seq_len, num_heads, head_dim] buffer and q_idx its row; k and
// v are device pointers (a KVCacheHIP's rows).
void BackendHIP::causal_attention(float* out, const float* q, std::size_t q_idx, const float* k, const float* v,
                                  std::size_t attend_len, std::size_t num_heads, std::size_t num_kv_heads,
                                  std::size_t head_dim, float scale)
{
    const char* qrow = reinterpret_cast<const char*>(q) + q_idx * num_heads * head_dim * elem();
    check(vvh_attention(out, qrow, k, v, 1, attend_len, num_heads, num_kv_heads, head_dim, scale, act_dtype(),
                        nullptr),
          "causal_attention");
}

// ---- KVCacheHIP ----
KVCacheHIP::KVCacheHIP(bool fp16) : fp16_(fp16) {}

KVCacheHIP::~KVCacheHIP()
{
    for (auto& l : layers_) {
        if (l.k) vvh_free(l.k);
        if (l.v) vvh_free(l.v);
    }
}

void KVCacheHIP::init(std::size_t num_layers, std::size_t kv_dim)
{
    if (!layers_.empty()) return;  // idempotent, as transformer_forward calls it every step
    kv_dim_ = kv_dim;
    seq_len_ = 0;
    layers_.resize(num_layers);
    reserve(reserve_tokens_);
}

void KVCacheHIP::grow(Layer& l, std::size_t tokens)
{
    const std::size_t bytes = tokens * kv_dim_ * elem();
    void* nk = nullptr;
    void* nv = nullptr;
    check(vvh_malloc(&nk, bytes), "kv cache");
    check(vvh_malloc(&nv, bytes), "kv cache");
    if (l.k && seq_len_) {
        check(vvh_memcpy_d2d(nk, l.k, seq_len_ * kv_dim_ * elem()), "kv cache grow");
        check(vvh_memcpy_d2d(nv, l.v, seq_len_ * kv_dim_ * elem()), "kv cache grow");
    }
    if (l.k) vvh_free(l.k);
    if (l.v) vvh_free(l.v);
    l.k = nk;
    l.v = nv;
    l.cap = tokens;
}

void KVCacheHIP::reserve(std::size_t tokens)
{
    reserve_tokens_ = tokens;
    for (auto& l : layers_)
        if (l.cap < tokens) grow(l, tokens);
}

void KVCacheHIP::append(std::size_t layer, const float* k, const float* v, std::size_t num_tokens)
{
    Layer& l = layers_.at(layer);
    if (seq_len_ + num_tokens > l.cap) grow(l, std::max(seq_len_ + num_tokens, 2 * l.cap));
    const std::size_t off = seq_len_ * kv_dim_ * elem(), n = num_tokens * kv_dim_ * elem();
    check(vvh_kv_append(static_cast<char*>(l.k) + off, static_cast<char*>(l.v) + off, k, v, n, nullptr), "kv append");
}

const float* KVCacheHIP::k(std::size_t layer) const
{
    return layer < layers_.size() ? static_cast<const float*>(layers_[layer].k) : nullptr;
}

const float* KVCacheHIP::v(std::size_t layer) const
{
    return layer < layers_.size() ? static_cast<const float*>(layers_[layer].v) : nullptr;
}

void KVCacheHIP::truncate(std::size_t new_seq_len)
{
    if (new_seq_len < seq_len_) seq_len_ = new_seq_len;
}

void* hip_device_allocate(std::size_t bytes)
{
    void* p = nullptr;
    check(vvh_pool_alloc(&p, bytes), "device_allocate");
    return p;
}

void hip_device_deallocate(void* ptr) { check(vvh_pool_free(ptr), "device_deallocate"); }
void hip_copy_h2d(void* d, const void* s, std::size_t n) { check(vvh_memcpy_h2d(d, s, n), "copy h2d"); }
void hip_copy_d2h(void* d, const void* s, std::size_t n) { check(vvh_memcpy_d2h(d, s, n), "copy d2h"); }
void hip_copy_d2d(void* d, const void* s, std::size_t n) { check(vvh_memcpy_d2d(d, s, n), "copy d2d"); }

}  // namespace vvllm
