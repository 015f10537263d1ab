// Auxiliary device kernels of the linear path: the per-channel quantizer,
// dtype conversion, and a counter-based normal generator for synthetic data.
#include <hip/hip_runtime.h>

#include "common.h"

namespace vvh {

typedef _Float16 f16;

// ---------------------------------------------------------------------------
// quantize_per_channel on the device (src/quantize/quantize.cc:9-48).
// One block per row.  The absmax uses the reference's comparison
// `std::max(absmax, |w|)` == (absmax < |w|) ? |w| : absmax, which ignores NaN;
// max is exact, so the reduction order cannot change the result.  The scale
// and its reciprocal are IEEE-correct fp32 divisions (this file is compiled
// with -fhip-fp32-correctly-rounded-divide-sqrt and without fast-math), the
// code is round-half-away-from-zero (roundf) of w * (1/scale), clamped with
// the reference's argument order so NaN becomes +127.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float ref_max(float a, float b) { return (a < b) ? b : a; }
__device__ __forceinline__ float ref_min(float a, float b) { return (b < a) ? b : a; }

// Source elements: fp32, or BF16 bits widened exactly to fp32 (the bits
// become the high half of the fp32 word, as the reference's loader does,
// src/safetensors/safetensors.cc:135-141).
__device__ __forceinline__ float src_f32(const float* w, int64_t i) { return w[i]; }
__device__ __forceinline__ float src_f32(const uint16_t* w, int64_t i)
{
    return __builtin_bit_cast(float, (uint32_t)w[i] << 16);
}

template <typename ST>
__global__ __launch_bounds__(256) void k_quantize(const ST* __restrict__ w, int64_t N, int64_t K,
                                                  int8_t* __restrict__ q, float* __restrict__ scales)
{
    __shared__ float part[4];
    __shared__ float row_scale;
    for (int64_t row = blockIdx.x; row < N; row += gridDim.x) {
        const ST* wr = w + row * K;
        float mx = 0.0f;
        for (int64_t k = threadIdx.x; k < K; k += 256) mx = ref_max(mx, __builtin_fabsf(src_f32(wr, k)));
        for (int off = 32; off > 0; off >>= 1) mx = ref_max(mx, __shfl_xor(mx, off));
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
        __syncthreads();
        if (threadIdx.x == 0) {
            float absmax = ref_max(ref_max(part[0], part[1]), ref_max(part[2], part[3]));
            const float scale = absmax / 127.0f;
            scales[row] = scale;
            row_scale = scale;
        }
        __syncthreads();
        const float scale = row_scale;
        int8_t* qr = q + row * K;
        if (scale == 0.0f) {
            for (int64_t k = threadIdx.x; k < K; k += 256) qr[k] = 0;
        } else {
            const float inv_scale = 1.0f / scale;
            for (int64_t k = threadIdx.x; k < K; k += 256) {
                float val = src_f32(wr, k) * inv_scale;
                val = ref_max(-128.0f, ref_min(127.0f, roundf(val)));
                qr[k] = (int8_t)val;
            }
        }
        __syncthreads();
    }
}

int launch_quantize(const void* w, int src_dtype, int64_t N, int64_t K, int8_t* q, float* scales, void* stream)
{
    const int64_t grid = N < 65536 ? N : 65536;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (src_dtype == VVH_BF16)
        hipLaunchKernelGGL(k_quantize<uint16_t>, dim3((unsigned)grid), dim3(256), 0, s,
                           static_cast<const uint16_t*>(w), N, K, q, scales);
    else
        hipLaunchKernelGGL(k_quantize<float>, dim3((unsigned)grid), dim3(256), 0, s,
                           static_cast<const float*>(w), N, K, q, scales);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// dtype conversion (round to nearest even), grid-stride.
// ---------------------------------------------------------------------------
template <typename DT, typename ST>
__global__ __launch_bounds__(256) void k_convert(DT* __restrict__ d, const ST* __restrict__ s, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        d[i] = (DT)(float)s[i];
}

int launch_convert(void* dst, int dst_dtype, const void* src, int src_dtype, int64_t n, void* stream)
{
    const int64_t want = (n + 255) / 256;
    const dim3 grid((unsigned)(want < 16384 ? (want > 0 ? want : 1) : 16384));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dst_dtype == VVH_F16 && src_dtype == VVH_F32)
        hipLaunchKernelGGL((k_convert<f16, float>), grid, dim3(256), 0, s, (f16*)dst, (const float*)src, n);
    else if (dst_dtype == VVH_F32 && src_dtype == VVH_F16)
        hipLaunchKernelGGL((k_convert<float, f16>), grid, dim3(256), 0, s, (float*)dst, (const f16*)src, n);
    else if (dst_dtype == VVH_F32)
        hipLaunchKernelGGL((k_convert<float, float>), grid, dim3(256), 0, s, (float*)dst, (const float*)src, n);
    else
        hipLaunchKernelGGL((k_convert<f16, f16>), grid, dim3(256), 0, s, (f16*)dst, (const f16*)src, n);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Synthetic N(mean, std) data: element i draws h = splitmix64(seed ^ i*phi),
// u1 = (top 24 bits + 0.5) / 2^24 in (0, 1), u2 = next 24 bits / 2^24, and
// takes the Box-Muller cosine branch in fp32.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

template <typename T>
__global__ __launch_bounds__(256) void k_fill_normal(T* __restrict__ d, int64_t n, uint64_t seed, float mean,
                                                     float std)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const uint64_t h = splitmix64(seed ^ ((uint64_t)i * 0x9E3779B97F4A7C15ull));
        const float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
        const float u2 = (float)((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
        d[i] = (T)(mean + std * z);
    }
}

// ---------------------------------------------------------------------------
// fp32 activations for the fp16 MFMA GEMM: row m of x [M, K] becomes row m of
// xs [M, 2K] fp16, the high parts hi_k = fp16(x_k * s) followed by the low
// parts lo_k = fp16(x_k * s - hi_k), with s = 2^p chosen per row so that the
// row's largest |x| * s lies in [2^14, 2^15) (in range for fp16 with room for
// its 11-bit significand), and rs[m] = 1/s.  x_k * s is exact (a power of
// two), x_k * s - hi_k is exact (Sterbenz), so hi + lo carries x_k * s to
// about 22 bits (or to the fp16 subnormal step 2^-24 of the scaled row); the
// int8 x fp16 products of both parts are exact in the GEMM's fp32
// accumulation.  A row without a finite nonzero maximum (all zeros, or
// containing Inf or NaN) keeps s = 1, so Inf and NaN reach the sums as such.
// One block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_split_f32(const float* __restrict__ x, int64_t K, f16* __restrict__ xs,
                                                   float* __restrict__ rs)
{
    __shared__ float part[4];
    const int64_t m = blockIdx.x;
    const float* xr = x + m * K;
    float mx = 0.0f;
    // an Inf or NaN anywhere in the row makes the row maximum Inf
    for (int64_t k = threadIdx.x; k < K; k += 256) {
        const float v = __builtin_fabsf(xr[k]);
        mx = __builtin_isfinite(v) ? fmaxf(mx, v) : __builtin_inff();
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    int p = 0;
    if (mx > 0.0f && __builtin_isfinite(mx)) {
        int e;
        (void)frexpf(mx, &e);          // mx = f * 2^e, f in [0.5, 1)
        p = 15 - e;                    // mx * 2^p in [2^14, 2^15)
        p = p < -126 ? -126 : (p > 126 ? 126 : p);
    }
    const float s = ldexpf(1.0f, p);
    if (threadIdx.x == 0) rs[m] = ldexpf(1.0f, -p);
    f16* hr = xs + m * 2 * K;
    for (int64_t k = threadIdx.x; k < K; k += 256) {
        const float v = xr[k] * s;
        const f16 hi = (f16)v;
        hr[k] = hi;
        hr[K + k] = __builtin_isfinite((float)hi) ? (f16)(v - (float)hi) : (f16)0.0f;
    }
}

int launch_split_f32(const float* x, int64_t M, int64_t K, void* xs, float* rs, void* stream)
{
    if (M <= 0) return 0;
    hipLaunchKernelGGL(k_split_f32, dim3((unsigned)M), dim3(256), 0, static_cast<hipStream_t>(stream), x, K,
                       static_cast<f16*>(xs), rs);
    return (int)hipGetLastError();
}

int launch_fill_normal(void* dst, int dtype, int64_t n, uint64_t seed, float mean, float std, void* stream)
{
    const int64_t want = (n + 255) / 256;
    const dim3 grid((unsigned)(want < 16384 ? (want > 0 ? want : 1) : 16384));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F32)
        hipLaunchKernelGGL((k_fill_normal<float>), grid, dim3(256), 0, s, (float*)dst, n, seed, mean, std);
    else
        hipLaunchKernelGGL((k_fill_normal<f16>), grid, dim3(256), 0, s, (f16*)dst, n, seed, mean, std);
    return (int)hipGetLastError();
}

}  // namespace vvh
