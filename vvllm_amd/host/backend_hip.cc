// BackendHIP implementation: C++20 host code over the C ABI of
// libvvllm_hip.so.  See backend_hip.h.
#include "backend_hip.h"

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

[[noreturn]] void outside_path(const char* op)
{
    throw std::logic_error(std::string("BackendHIP::") + op +
                           " is outside the int8 linear path this backend implements");
}

}  // namespace

BackendHIP::BackendHIP(bool fp16, int device) : fp16_(fp16)
{
    char name[256] = {0};
    check(vvh_init(device, name, sizeof(name)), "init");
    name_ = name;
}

BackendHIP::~BackendHIP() = default;

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
    return static_cast<const int8_t*>(host_rows);
}

void BackendHIP::forget_weight(const int8_t* host_weight)
{
    vvh_weight h = 0;
    if (vvh_weight_find(host_weight, &h) == VVH_OK) check(vvh_weight_release(h), "forget_weight");
}

void BackendHIP::matmul(float*, const float*, const float*, std::size_t, std::size_t, std::size_t) { outside_path("matmul"); }
void BackendHIP::add(float*, const float*, const float*, std::size_t) { outside_path("add"); }
void BackendHIP::mul(float*, const float*, const float*, std::size_t) { outside_path("mul"); }
void BackendHIP::silu(float*, const float*, std::size_t) { outside_path("silu"); }
void BackendHIP::rms_norm(float*, const float*, const float*, std::size_t, float) { outside_path("rms_norm"); }
void BackendHIP::softmax(float*, const float*, std::size_t) { outside_path("softmax"); }
void BackendHIP::rope(float*, float*, std::size_t, std::size_t, std::size_t, std::size_t, std::size_t, float) { outside_path("rope"); }
void BackendHIP::linear(float*, const float*, const float*, const float*, std::size_t, std::size_t, std::size_t) { outside_path("linear"); }
void BackendHIP::silu_mul(float*, const float*, const float*, std::size_t) { outside_path("silu_mul"); }
void BackendHIP::linear_add(float*, const float*, const float*, const float*, const float*, std::size_t, std::size_t, std::size_t) { outside_path("linear_add"); }
void BackendHIP::embedding(float*, const float*, std::size_t, std::size_t, std::size_t) { outside_path("embedding"); }
void BackendHIP::causal_attention(float*, const float*, std::size_t, const float*, const float*, std::size_t, std::size_t, std::size_t, std::size_t, float) { outside_path("causal_attention"); }

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
