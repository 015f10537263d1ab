// C-ABI shim over the reference's own CPU code -- TEST INFRASTRUCTURE ONLY.
//
// oracle/Makefile compiles this file together with the reference's
// src/backend/backend_naive.cc and src/quantize/quantize.cc, read in place
// from the reference tree (nothing is copied), into oracle/_ref/.  The
// result is the reference's BackendCPU::linear_q8 / linear_q8_add and
// quantize_per_channel, callable through ctypes, used to check the oracle's
// restatement bit-for-bit and to write the golden vectors.
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

}  // extern "C"
