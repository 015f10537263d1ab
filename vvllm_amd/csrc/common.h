// Internal declarations shared by the runtime and the kernels of
// libvvllm_hip.so.  Nothing here is part of the public C ABI
// (include/vvllm_hip.h).
#pragma once

#include <cstddef>
#include <cstdint>

#include "vvllm_hip.h"

namespace vvh {

// One linear_q8 problem as the kernels see it.  All pointers are device
// pointers; `inp`/`out`/`res` carry the element types the launcher was
// instantiated for.  Sizes are 64-bit: a single weight may exceed 2^31 codes
// on a 288 GB device.
struct LinArgs {
    void* out;
    const void* inp;
    const void* res;          // may be null; may alias out
    const int8_t* w;          // [N, K] codes
    const float* scales;      // [N]
    const float* bias;        // [N] or null
    int64_t M, N, K;
    int32_t ksplit;           // decode kernels: waves cooperating on one 16-row tile (1, 2, 4)
    int32_t block_begin;      // grouped launch: first block of this problem
};

// Kernel families (values match vvh_kernel).
enum Kernel : int {
    K_AUTO = VVH_KERNEL_AUTO,
    K_GENERIC = VVH_KERNEL_GENERIC,
    K_GEMV_F32 = VVH_KERNEL_GEMV_F32,
    K_SKINNY = VVH_KERNEL_SKINNY,
    K_GEMM = VVH_KERNEL_GEMM,
};

// Largest M served by the decode kernels.
constexpr int64_t kSkinnyMaxM = 16;   // one 16-row MFMA operand
constexpr int64_t kGemvF32MaxM = 8;   // rows of fp32 activations per pass

// Rows of output channels handled by one wave of the decode kernels.
constexpr int kDecodeTileN = 16;

// Number of blocks a decode-kernel launch needs for one problem.
inline int64_t decode_blocks(const LinArgs& a)
{
    const int64_t tiles = (a.N + kDecodeTileN - 1) / kDecodeTileN;
    const int64_t tiles_per_block = 4 / a.ksplit;
    return (tiles + tiles_per_block - 1) / tiles_per_block;
}

// GEMM tile shape.
constexpr int kGemmBM = 128;
constexpr int kGemmBN = 128;
constexpr int kGemmBK = 64;

// Launchers (linear_kernels.hip).  Return a hipError_t value as int.
int launch_generic(const LinArgs& a, int act, int out, void* stream);
int launch_gemv_f32(const LinArgs& a, int out, void* stream);
int launch_skinny(const LinArgs& a, int out, void* stream);
int launch_skinny_grouped(const LinArgs* dev_table, int count, int64_t total_blocks, int out,
                          void* stream);
int launch_gemm(const LinArgs& a, int out, void* stream);

// Auxiliary kernels (aux_kernels.hip).
int launch_quantize(const float* w, int64_t N, int64_t K, int8_t* q, float* scales, void* stream);
int launch_convert(void* dst, int dst_dtype, const void* src, int src_dtype, int64_t n,
                   void* stream);
int launch_fill_normal(void* dst, int dtype, int64_t n, uint64_t seed, float mean, float std,
                       void* stream);

}  // namespace vvh
