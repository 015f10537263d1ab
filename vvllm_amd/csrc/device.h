// Device-side building blocks shared by the int8 linear kernels
// (linear_kernels.hip): vector types, the exact int8 -> fp16
// code conversion, pipeline synchronisation helpers, address-space casts,
// the XCD-aware block remap and the 32x32x16 MFMA fragment reader/multiplier
// of the LDS-staged GEMMs.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace vvh {

typedef _Float16 f16;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float ld_f(const T* p) { return (float)*p; }

template <typename T>
__device__ __forceinline__ void st_f(T* p, float v) { *p = (T)v; }

// Four int8 codes (one dword, little-endian k order) -> four exact fp16
// values in two dwords.  The code is biased to u = q + 128 in [0, 255] and
// placed in the low mantissa byte of an fp16 with exponent 2^10
// (0x6400 | u == 1024 + u exactly); subtracting 1152 = 1024 + 128 returns q.
__device__ __forceinline__ void i8x4_to_f16x4(uint32_t d, uint32_t& lo, uint32_t& hi)
{
    const uint32_t u = d ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // bytes 0,1
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes 2,3
    const h2 off = {(f16)1152.0f, (f16)1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, a) - off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, b) - off);
}

// 16 codes -> two 8-wide fp16 MFMA operands (codes 0-7 and 8-15).
__device__ __forceinline__ void i8x16_to_h8x2(const u4 w, h8& b0, h8& b1)
{
    uint32_t c[8];
    i8x4_to_f16x4(w[0], c[0], c[1]);
    i8x4_to_f16x4(w[1], c[2], c[3]);
    i8x4_to_f16x4(w[2], c[4], c[5]);
    i8x4_to_f16x4(w[3], c[6], c[7]);
    b0 = __builtin_bit_cast(h8, u4{c[0], c[1], c[2], c[3]});
    b1 = __builtin_bit_cast(h8, u4{c[4], c[5], c[6], c[7]});
}

// 8 codes (two dwords) -> one 8-wide fp16 MFMA operand, in code order.
__device__ __forceinline__ h8 i8x8_to_h8(const uint32_t w0, const uint32_t w1)
{
    uint32_t c[4];
    i8x4_to_f16x4(w0, c[0], c[1]);
    i8x4_to_f16x4(w1, c[2], c[3]);
    return __builtin_bit_cast(h8, u4{c[0], c[1], c[2], c[3]});
}

// One step of merging decode-attention partials: a partial with running
// maximum mi (log2 units), exponential sum li and numerator oi joins the
// totals (num, den) under the common maximum M.  The attention kernel's merge
// of its waves and the o-projection's merge stage (k_dot input stage 3) both
// take it, in part order, so the two produce the same bits.
__device__ __forceinline__ void attn_merge_add(float& num, float& den, float mi, float M, float oi, float li)
{
    const float f = exp2f(mi - M);
    num = __builtin_fmaf(f, oi, num);
    den = __builtin_fmaf(f, li, den);
}

// LDS reads done (lgkmcnt(0)), then s_barrier, without waiting on vector
// memory loads.  Written with builtins so the compiler's wait-count tracking
// sees the lgkmcnt(0); the empty asm with a memory clobber keeps the
// compiler from moving memory accesses across the barrier.
// The scheduling barriers keep the instruction scheduler from hoisting work
// of the next pipeline step (which only depends on registers) above it.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // vmcnt 63, expcnt 7: no wait; lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// Block-wide sum over 256 threads (4 waves); `red` holds 4 floats.  Shared by
// k_rms_norm and the RMSNorm input stage of k_dot, which must round alike.
__device__ __forceinline__ float block_sum256(float v, float* red)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// RMSNorm's sum of squares in one wave, the order k_rms_norm and k_dot's
// RMSNorm input stages share: lane l takes the chunks l, l + 64, l + 128, ...
// of 8 consecutive values and adds their squares in order (values past the
// row add an exact 0), then the wave adds its lanes with an xor butterfly,
// which leaves every lane with the same bits (each step adds the same two
// numbers on both partner lanes).  One wave holds the whole sum, so a block
// needs no barrier for it.
__device__ __forceinline__ float rms_sumsq8(float ss, const float (&v)[8])
{
#pragma unroll
    for (int e = 0; e < 8; e++) ss = __builtin_fmaf(v[e], v[e], ss);
    return ss;
}
__device__ __forceinline__ float rms_sumsq_h8(float ss, const h8 x, bool ok)
{
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = ok ? (float)x[e] : 0.0f;
    return rms_sumsq8(ss, v);
}
// Sum over the wave, every lane getting the same bits: group_sum(v, 64)
// (pairs of lanes 1, 2, 4, 8 apart within rows of 16 as DPP moves, then the
// four row sums as (R0 + R1) + (R2 + R3) through row broadcasts and a lane
// read, no LDS-pipeline round trip).
__device__ __forceinline__ float wave_sum_xor(float v);

// RMSNorm's divisor and output, and the SiLU-gated product, in the
// reference's fp32 operation order (backend_naive.cc:68-76, :297-298); used by
// the standalone kernels and by the fused input stage of k_dot alike.  The
// products are materialised as fp32 (the empty asm) before any conversion to
// fp16: otherwise the compiler may fold multiply and conversion into one
// v_fma_mixlo_f16, which rounds once to fp16, in one kernel and not in
// another, and the two then disagree by one fp16 ulp wherever rounding to
// fp32 first changes the result.
__device__ __forceinline__ float rms_of(float sum_sq, int64_t n, float eps) { return sqrtf(sum_sq / (float)n + eps); }
__device__ __forceinline__ float rms_apply(float x, float rms, float w)
{
    float r = x / rms * w;
    __asm__("" : "+v"(r));
    return r;
}
__device__ __forceinline__ float silu_mul_ref(float g, float u)
{
    float r = (g / (1.0f + expf(-g))) * u;
    __asm__("" : "+v"(r));
    return r;
}

// Split-half RoPE of one pair (x0, x1) = (v[i], v[i + D/2]) of a head at
// position p, in the reference's operation order (backend_naive.cc:93-137):
// angle = p * (1 / theta^(2i/D)) with the power, cos and sin taken in fp64
// and rounded to fp32.  The four products are rounded to fp32 before the sum
// and the difference (the empty asm: otherwise the compiler may fuse them
// into FMAs in one kernel and not in another), so k_rope and the RoPE
// epilogue of a q/k/v plan rotate bit-identically.
// rope_freq gives the pair's frequency (an fp64 power: the longest part, and
// the same at every position, so plans keep a table of it), rope_cs_freq
// the cosine and sine at position p (one fp64 argument reduction for both),
// rope_apply the rotation; rope_rotate is the three in turn.
__device__ __forceinline__ float rope_freq(int64_t i, int64_t D, float theta)
{
    const float e = (float)(2 * i) / (float)D;
    return 1.0f / (float)pow((double)theta, (double)e);
}
__device__ __forceinline__ void rope_cs_freq(int64_t p, float freq, float& c, float& sn)
{
    const float angle = (float)p * freq;
    double sd, cd;
    sincos((double)angle, &sd, &cd);
    c = (float)cd;
    sn = (float)sd;
}
__device__ __forceinline__ void rope_cs(int64_t p, int64_t i, int64_t D, float theta, float& c, float& sn)
{
    rope_cs_freq(p, rope_freq(i, D, theta), c, sn);
}
__device__ __forceinline__ void rope_apply(float x0, float x1, float c, float sn, float& r0, float& r1)
{
    float a = x0 * c, b = x1 * sn, d = x0 * sn, f = x1 * c;
    __asm__("" : "+v"(a), "+v"(b), "+v"(d), "+v"(f));
    r0 = a - b;
    r1 = d + f;
}
__device__ __forceinline__ void rope_rotate(float x0, float x1, int64_t p, int64_t i, int64_t D, float theta,
                                            float& r0, float& r1)
{
    float c, sn;
    rope_cs(p, i, D, theta, c, sn);
    rope_apply(x0, x1, c, sn, r0, r1);
}

// Butterfly steps within rows of 16 lanes as DPP moves (one VALU op, no
// LDS-pipeline round trip like __shfl_xor): quad_perm [1,0,3,2] and
// [2,3,0,1] exchange with lanes l^1 and l^2; row_half_mirror (lane i <-> 7-i
// of each 8) and row_mirror (i <-> 15-i of each 16) reach the other half
// once the smaller groups already hold equal values.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// The values of lanes l & ~16 and l | 16 (p16) or l & ~32 and l | 32 (p32),
// lower lane first, in every lane: v_permlane16_swap / v_permlane32_swap with
// both operands the same register (one VALU op each, no LDS-pipeline round
// trip).  a + b over them is the xor-16 / xor-32 shuffle sum with its
// operands in a fixed order: each addition commutes, so the bits are the same.
__device__ __forceinline__ void lanes_x16(float v, float& lo, float& hi)
{
    const int vi = __builtin_bit_cast(int, v);
    const auto q = __builtin_amdgcn_permlane16_swap(vi, vi, false, false);
    lo = __builtin_bit_cast(float, (int)q[0]);
    hi = __builtin_bit_cast(float, (int)q[1]);
}
__device__ __forceinline__ void lanes_x32(float v, float& lo, float& hi)
{
    const int vi = __builtin_bit_cast(int, v);
    const auto q = __builtin_amdgcn_permlane32_swap(vi, vi, false, false);
    lo = __builtin_bit_cast(float, (int)q[0]);
    hi = __builtin_bit_cast(float, (int)q[1]);
}
__device__ __forceinline__ float sum_x16(float v)
{
    float lo, hi;
    lanes_x16(v, lo, hi);
    return lo + hi;
}
__device__ __forceinline__ float sum_x32(float v)
{
    float lo, hi;
    lanes_x32(v, lo, hi);
    return lo + hi;
}
__device__ __forceinline__ float max_x16(float v)
{
    float lo, hi;
    lanes_x16(v, lo, hi);
    return fmaxf(lo, hi);
}
__device__ __forceinline__ float max_x32(float v)
{
    float lo, hi;
    lanes_x32(v, lo, hi);
    return fmaxf(lo, hi);
}

// Sum / max over aligned groups of L lanes (L = 1, 2, 4, ..., 64,
// wave-uniform); every lane of a group gets the group's result.  DPP steps
// within rows of 16, lane swaps across rows.  All lanes must be active.
// L = 64 adds the row sums as the xor-16 and xor-32 shuffles would, (R0 +
// R1) + (R2 + R3) (each addition commutes, so the bits are the same), from
// row_bcast15 (rows 1 and 3 add lane 15 of rows 0 and 2) and row_bcast31
// (row 3 adds lane 31), then lane 63 read into a scalar register.
__device__ __forceinline__ float group_sum(float v, int L)
{
    if (L >= 2) v += dpp_mov<0xB1>(v);
    if (L >= 4) v += dpp_mov<0x4E>(v);
    if (L >= 8) v += dpp_mov<0x141>(v);
    if (L >= 16) v += dpp_mov<0x140>(v);
    if (L >= 64) {
        const int vi = __builtin_bit_cast(int, v);
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, vi, 0x142, 0xA, 0xF, false));
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF,
                                                                   false));
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    }
    if (L >= 32) v = sum_x16(v);
    return v;
}
__device__ __forceinline__ float wave_sum_xor(float v) { return group_sum(v, 64); }
__device__ __forceinline__ float group_max(float v, int L)
{
    if (L >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));
    if (L >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));
    if (L >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
    if (L >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
    if (L >= 32) v = max_x16(v);
    if (L >= 64) v = max_x32(v);
    return v;
}

// Pointers read from memory (plan tables) are generic to the compiler, which
// then emits flat loads; those count in lgkmcnt as well as vmcnt, so every
// wait on a scalar load would also drain the weight stream.  Kernels that
// take their pointers from tables cast them to the global address space.
#define VVH_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const VVH_GLOBAL T* gbl(const T* p)
{
    return (const VVH_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ VVH_GLOBAL T* gbl(T* p)
{
    return (VVH_GLOBAL T*)p;
}

// Plan tables are read-only for the whole launch.  Reading them through the
// constant address space lets the compiler use scalar loads (lgkmcnt) even
// though the kernel stores to global memory; otherwise it cannot rule out
// aliasing and reads them with vector loads that join the weight stream's
// vmcnt queue.
#define VVH_CONST __attribute__((address_space(4)))
template <typename T>
__device__ __forceinline__ const VVH_CONST T* cst(const T* p)
{
    return (const VVH_CONST T*)p;
}

__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t total)
{
    constexpr int64_t X = 8;
    const int64_t per = total / X, rem = total % X;
    const int64_t xcd = b % X, idx = b / X;
    return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
}

// s_waitcnt with vmcnt <= v (expcnt, lgkmcnt not waited on); gfx9 encoding.
template <int V>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(V >= 0 && V < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((V & 15) | ((V >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS layout of a GEMM stage (1 KB per 64-lane load instruction, lane i ->
// bytes 16i..16i+15; the swizzles put the 16 rows read by 16 lanes of one
// 16-byte fragment load in 16 distinct 16-byte bank groups of the LDS):
//   A: 128 rows x 128 B; row r keeps 16-byte chunk c at slot c ^ ((r >> 1) & 7)
//   B: rows of 64 B;     row r keeps 16-byte chunk c at slot c ^ ((r >> 2) & 3)
__device__ __forceinline__ int swz_a(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int swz_b(int r, int c) { return c ^ ((r >> 2) & 3); }

}  // namespace vvh
