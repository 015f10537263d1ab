// Device tags of the vvllm tensor layer, with a HIP member.
// Mirrors include/vvllm/tensor/device.h:6-10 of the reference (CPU, CUDA);
// HIP is the tag BackendHIP::device() returns, so Tensor memory for it is
// routed to the caching allocator of libvvllm_hip (vvh_pool_alloc).
#pragma once

namespace vvllm
{

enum class Device
{
    CPU,
    CUDA,
    HIP
};

}  // namespace vvllm
