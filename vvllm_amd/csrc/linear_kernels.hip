// INT8 per-channel linear kernels for gfx950 (CDNA4, wave64).
//
//   out[m, n] = (sum_k x[m, k] * q[n, k]) * scale[n] + bias[n] (+ res[m, n])
//
// Semantics follow Backend::linear_q8 / linear_q8_add
// (include/vvllm/backend/backend.h:62-65, :75-78): the dot product is taken
// over the exact int8 codes with fp32 accumulation and the per-channel scale
// is applied afterwards, as BackendCPU does (src/backend/backend_naive.cc:
// 216-288).  The codes are never pre-multiplied by the scale (the
// reference's CUDA path does, rounding q*scale to fp16,
// src/backend/cuda_kernels.cu:804-814): int8 -> fp16 of a raw code is exact,
// so MFMA products are exact and only the fp32 accumulation rounds.
//
// Kernel families:
//   k_generic   any shape/alignment; one thread per output, sequential k.
//   k_gemv_f32  fp32 activations, M <= 8 per pass: VALU fp32 FMAs.
//   k_skinny    fp16 activations, M <= 16: one wave owns 16 output channels,
//               streams their int8 rows with 16-byte loads, converts codes to
//               fp16 in registers and accumulates with
//               v_mfma_f32_16x16x32_f16 (the 16 activation rows are the MFMA
//               M side, so no cross-lane reduction is needed).
//   k_gemm      fp16 activations, M > 16: 128x128x64 LDS tiles, int8 -> fp16
//               on the way into LDS, v_mfma_f32_32x32x16_f16, fp32 accumulate,
//               fused scale/bias/residual epilogue.
#include <hip/hip_runtime.h>

#include "common.h"

namespace vvh {

typedef _Float16 f16;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
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

// Epilogue for one output element, in fp32, one rounding to OT.
template <typename OT>
__device__ __forceinline__ void store_out(const LinArgs& a, int64_t m, int64_t n, float acc)
{
    float v = acc * a.scales[n];
    if (a.bias) v += a.bias[n];
    const int64_t o = m * a.N + n;
    if (a.res) v += ld_f(static_cast<const OT*>(a.res) + o);
    st_f(static_cast<OT*>(a.out) + o, v);
}

// Weight rows are streamed exactly once: load them non-temporally so they do
// not evict the activations from the caches.
__device__ __forceinline__ u4 ld_stream(const int8_t* p)
{
    return __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
}

// ---------------------------------------------------------------------------
// generic: any M, N, K, alignment, dtypes.  One thread per output element.
// ---------------------------------------------------------------------------
template <typename AT, typename OT>
__global__ __launch_bounds__(256) void k_generic(LinArgs a)
{
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.M * a.N) return;
    const int64_t m = idx / a.N;
    const int64_t n = idx - m * a.N;
    const AT* x = static_cast<const AT*>(a.inp) + m * a.K;
    const int8_t* w = a.w + n * a.K;
    float acc = 0.0f;
    for (int64_t k = 0; k < a.K; k++) acc = __builtin_fmaf((float)x[k], (float)w[k], acc);
    store_out<OT>(a, m, n, acc);
}

// ---------------------------------------------------------------------------
// Decode kernels share one work decomposition.  A block is 4 waves.  A tile
// is 16 consecutive output channels; `ksplit` waves of a block cooperate on
// one tile, each taking a contiguous share of its 64-wide k steps, so a block
// covers 4/ksplit tiles.  Within a wave, lane l reads the 16 codes
// w[n0 + l%16][64*s + 16*(l/16) .. +16] at step s: 16 rows x 64 contiguous
// bytes per instruction.
// ---------------------------------------------------------------------------
struct DecodeCoord {
    int lane, wave, ks, ksplit;
    int64_t tile;
    int64_t s0, s1;  // k-step range [s0, s1) of this wave
};

__device__ __forceinline__ DecodeCoord decode_coord(const LinArgs& a, int64_t block)
{
    DecodeCoord c;
    c.lane = threadIdx.x & 63;
    c.wave = threadIdx.x >> 6;
    c.ksplit = a.ksplit;
    c.ks = c.wave % c.ksplit;
    c.tile = block * (4 / c.ksplit) + c.wave / c.ksplit;
    const int64_t steps = (a.K + 63) / 64;
    const int64_t per = (steps + c.ksplit - 1) / c.ksplit;
    c.s0 = c.ks * per;
    c.s1 = c.s0 + per < steps ? c.s0 + per : steps;
    return c;
}

// ---------------------------------------------------------------------------
// k_gemv_f32: fp32 activations.  Each lane accumulates MT rows of fp32 dot
// products over its 16-code chunks with exact int8 -> fp32 conversion and
// fp32 FMAs; the four lanes sharing a channel are combined with cross-lane
// adds, then the ksplit waves through LDS.  blockIdx.y selects the group of
// MT activation rows.
// ---------------------------------------------------------------------------
template <int MT, typename OT>
__device__ __forceinline__ void gemv_f32_body(const LinArgs& a, int64_t block, int64_t mbase)
{
    __shared__ float red[4][MT][16];
    const DecodeCoord c = decode_coord(a, block);
    const int64_t n0 = c.tile * kDecodeTileN;
    const int64_t n = n0 + (c.lane & 15);
    const int64_t nrow = n < a.N ? n : a.N - 1;
    const int chunk = c.lane >> 4;
    const int8_t* wp = a.w + nrow * a.K + chunk * 16;
    const float* x = static_cast<const float*>(a.inp);

    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) acc[m] = 0.0f;

    if (n0 < a.N) {
#pragma unroll 2
        for (int64_t s = c.s0; s < c.s1; s++) {
            const int64_t k = s * 64 + chunk * 16;
            if (k < a.K) {
                const u4 wv = ld_stream(wp + s * 64);
                float wf[16];
#pragma unroll
                for (int j = 0; j < 4; j++) {
#pragma unroll
                    for (int b = 0; b < 4; b++)
                        wf[4 * j + b] = (float)(int8_t)((wv[j] >> (8 * b)) & 0xff);
                }
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    if (mbase + m < a.M) {
                        const f4* xp = reinterpret_cast<const f4*>(x + (mbase + m) * a.K + k);
                        float sum = acc[m];
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const f4 xv = xp[q];
                            sum = __builtin_fmaf(xv[0], wf[4 * q + 0], sum);
                            sum = __builtin_fmaf(xv[1], wf[4 * q + 1], sum);
                            sum = __builtin_fmaf(xv[2], wf[4 * q + 2], sum);
                            sum = __builtin_fmaf(xv[3], wf[4 * q + 3], sum);
                        }
                        acc[m] = sum;
                    }
                }
            }
        }
    }
    // combine the four 16-byte chunks of each channel (lanes l, l^16, l^32, l^48)
#pragma unroll
    for (int m = 0; m < MT; m++) {
        acc[m] += __shfl_xor(acc[m], 16);
        acc[m] += __shfl_xor(acc[m], 32);
    }
    if (c.ksplit > 1) {
        if (c.lane < 16) {
#pragma unroll
            for (int m = 0; m < MT; m++) red[c.wave][m][c.lane] = acc[m];
        }
        __syncthreads();
        if (c.ks == 0 && c.lane < 16) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                float s = red[c.wave][m][c.lane];
                for (int j = 1; j < c.ksplit; j++) s += red[c.wave + j][m][c.lane];
                acc[m] = s;
            }
        }
    }
    if (c.ks == 0 && c.lane < 16 && n < a.N) {
#pragma unroll
        for (int m = 0; m < MT; m++)
            if (mbase + m < a.M) store_out<OT>(a, mbase + m, n, acc[m]);
    }
}

template <int MT, typename OT>
__global__ __launch_bounds__(256) void k_gemv_f32(LinArgs a)
{
    gemv_f32_body<MT, OT>(a, blockIdx.x, (int64_t)blockIdx.y * MT);
}

// ---------------------------------------------------------------------------
// k_skinny: fp16 activations, M <= 16, MFMA 16x16x32.
//   A operand (16 x 32): lane l holds x[m = l%16][kslot 8*(l/16) .. +8]
//   B operand (32 x 16): lane l holds q[n0 + l%16][kslot 8*(l/16) .. +8]
//   D (16 x 16):         lane l, reg r = acc[m = 4*(l/16) + r][n0 + l%16]
// A 16-byte chunk of 16 codes feeds two MFMAs (codes 0-7, then 8-15); the
// activations are read with the same k mapping, so the sum is unchanged.
// Lanes whose row m >= M feed zeros.
// ---------------------------------------------------------------------------
template <typename OT>
__device__ __forceinline__ void skinny_body(const LinArgs& a, int64_t block)
{
    __shared__ f4 red[4][64];
    const DecodeCoord c = decode_coord(a, block);
    const int64_t n0 = c.tile * kDecodeTileN;
    const int64_t nrow = n0 + (c.lane & 15) < a.N ? n0 + (c.lane & 15) : a.N - 1;
    const int chunk = c.lane >> 4;
    const int m = c.lane & 15;
    const bool mvalid = m < a.M;
    const int8_t* wp = a.w + nrow * a.K + chunk * 16;
    const f16* xp = static_cast<const f16*>(a.inp) + (mvalid ? m : 0) * a.K + chunk * 16;

    f4 acc0 = {0.f, 0.f, 0.f, 0.f};
    f4 acc1 = {0.f, 0.f, 0.f, 0.f};
    if (n0 < a.N) {
        constexpr int U = 8;
        int64_t s = c.s0;
        const int64_t kfull = a.K / 64;  // steps whose 64 codes are all in range
        // main loop: U full steps per batch, loads first
        for (; s + U <= c.s1 && s + U <= kfull; s += U) {
            u4 wv[U];
            h8 xa[U], xb[U];
#pragma unroll
            for (int u = 0; u < U; u++) wv[u] = ld_stream(wp + (s + u) * 64);
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (mvalid) {
                    xa[u] = *reinterpret_cast<const h8*>(xp + (s + u) * 64);
                    xb[u] = *reinterpret_cast<const h8*>(xp + (s + u) * 64 + 8);
                } else {
                    xa[u] = h8{};
                    xb[u] = h8{};
                }
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                h8 b0, b1;
                i8x16_to_h8x2(wv[u], b0, b1);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[u], b0, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xb[u], b1, acc1, 0, 0, 0);
            }
        }
        // remainder steps (including a partial last step when K % 64 != 0)
        for (; s < c.s1; s++) {
            const int64_t k = s * 64 + chunk * 16;
            u4 wv = {0u, 0u, 0u, 0u};
            h8 xa = {}, xb = {};
            if (k < a.K) {
                wv = ld_stream(wp + s * 64);
                if (mvalid) {
                    xa = *reinterpret_cast<const h8*>(xp + s * 64);
                    xb = *reinterpret_cast<const h8*>(xp + s * 64 + 8);
                }
            }
            h8 b0, b1;
            i8x16_to_h8x2(wv, b0, b1);
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, b0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xb, b1, acc1, 0, 0, 0);
        }
    }
    f4 acc = acc0 + acc1;
    if (c.ksplit > 1) {
        red[c.wave][c.lane] = acc;
        __syncthreads();
        if (c.ks == 0) {
            for (int j = 1; j < c.ksplit; j++) acc += red[c.wave + j][c.lane];
        }
    }
    if (c.ks == 0) {
        const int64_t n = n0 + (c.lane & 15);
        if (n < a.N) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t mm = 4 * (c.lane >> 4) + r;
                if (mm < a.M) store_out<OT>(a, mm, n, acc[r]);
            }
        }
    }
}

template <typename OT>
__global__ __launch_bounds__(256) void k_skinny(LinArgs a)
{
    skinny_body<OT>(a, blockIdx.x);
}

// Grouped launch: block b serves problem p with
// table[p].block_begin <= b < table[p+1].block_begin.
template <typename OT>
__global__ __launch_bounds__(256) void k_skinny_grouped(const LinArgs* __restrict__ table, int count)
{
    const int b = blockIdx.x;
    int lo = 0, hi = count - 1;
    while (lo < hi) {  // last p with block_begin <= b
        const int mid = (lo + hi + 1) >> 1;
        if (table[mid].block_begin <= b) lo = mid;
        else hi = mid - 1;
    }
    const LinArgs a = table[lo];
    skinny_body<OT>(a, b - a.block_begin);
}

// ---------------------------------------------------------------------------
// k_gemm: fp16 activations, M > 16.
// Block tile 128(m) x 128(n) x 64(k), 256 threads = 4 waves in a 2x2 grid,
// each wave 64x64 = 2x2 MFMA 32x32x16 tiles.
//   A operand (32 x 16): lane l holds x[i = l%32][kslot 8*(l/32) .. +8]
//   B operand (16 x 32): lane l holds q[j = l%32][kslot 8*(l/32) .. +8]
//   D (32 x 32): lane l, reg r = acc[i = 8*(r/4) + 4*(l/32) + r%4][j = l%32]
// Stages are double-buffered in LDS (fp16, row stride 72 halves = 144 B so
// the 16-byte fragment reads of 8 consecutive rows hit distinct banks).
// The next stage's global loads are issued before the current stage's MFMAs.
// Blocks are remapped so that consecutive tiles land on one XCD (block ids
// are dealt to the 8 XCDs round-robin), m-fastest: an XCD streams a band of
// weight columns once and re-reads the (small) activations from its L2.
// ---------------------------------------------------------------------------
constexpr int kLdsStride = kGemmBK + 8;

__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t total)
{
    constexpr int64_t X = 8;
    const int64_t per = total / X, rem = total % X;
    const int64_t xcd = b % X, idx = b / X;
    return (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
}

template <typename OT>
__global__ __launch_bounds__(256) void k_gemm(LinArgs a)
{
    __shared__ __attribute__((aligned(16))) f16 As[2][kGemmBM][kLdsStride];
    __shared__ __attribute__((aligned(16))) f16 Bs[2][kGemmBN][kLdsStride];

    const int64_t nbm = (a.M + kGemmBM - 1) / kGemmBM;
    const int64_t nbn = (a.N + kGemmBN - 1) / kGemmBN;
    const int64_t logical = xcd_remap(blockIdx.x, nbm * nbn);
    const int64_t m0 = (logical % nbm) * kGemmBM;
    const int64_t n0 = (logical / nbm) * kGemmBN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const f16* X = static_cast<const f16*>(a.inp);

    // loader coordinates: A 4 x 16 B chunks per thread, B 2 x 16 B chunks
    int a_row[4], a_kc[4];
    bool a_ok[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int cidx = tid + 256 * i;
        a_row[i] = cidx >> 3;
        a_kc[i] = (cidx & 7) * 8;
        a_ok[i] = m0 + a_row[i] < a.M;
    }
    int b_row[2], b_kc[2];
    bool b_ok[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int cidx = tid + 256 * i;
        b_row[i] = cidx >> 2;
        b_kc[i] = (cidx & 3) * 16;
        b_ok[i] = n0 + b_row[i] < a.N;
    }

    u4 ra[4], rb[2];
    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t k = k0 + a_kc[i];
            ra[i] = (a_ok[i] && k < a.K)
                        ? *reinterpret_cast<const u4*>(X + (m0 + a_row[i]) * a.K + k)
                        : u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int64_t k = k0 + b_kc[i];
            rb[i] = (b_ok[i] && k < a.K) ? ld_stream(a.w + (n0 + b_row[i]) * a.K + k)
                                         : u4{0u, 0u, 0u, 0u};
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<u4*>(&As[buf][a_row[i]][a_kc[i]]) = ra[i];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            h8 b0, b1;
            i8x16_to_h8x2(rb[i], b0, b1);
            *reinterpret_cast<h8*>(&Bs[buf][b_row[i]][b_kc[i]]) = b0;
            *reinterpret_cast<h8*>(&Bs[buf][b_row[i]][b_kc[i] + 8]) = b1;
        }
    };

    f16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f16v{};

    const int64_t nk = (a.K + kGemmBK - 1) / kGemmBK;
    gload(0);
    lstore(0);
    __syncthreads();

    const int fr = lane & 31;         // fragment row within a 32-row sub-tile
    const int fk = (lane >> 5) * 8;   // fragment k offset within a 16-wide k slice
    for (int64_t kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * kGemmBK);
#pragma unroll
        for (int kk = 0; kk < kGemmBK; kk += 16) {
            h8 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                fa[i] = *reinterpret_cast<const h8*>(&As[buf][wm * 64 + i * 32 + fr][kk + fk]);
#pragma unroll
            for (int j = 0; j < 2; j++)
                fb[j] = *reinterpret_cast<const h8*>(&Bs[buf][wn * 64 + j * 32 + fr][kk + fk]);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int64_t n = n0 + wn * 64 + j * 32 + (lane & 31);
        if (n >= a.N) continue;
        const float sc = a.scales[n];
        const float bi = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t mm = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (mm < a.M) {
                    float v = acc[i][j][r] * sc + bi;
                    const int64_t o = mm * a.N + n;
                    if (a.res) v += ld_f(static_cast<const OT*>(a.res) + o);
                    st_f(static_cast<OT*>(a.out) + o, v);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

int launch_generic(const LinArgs& a, int act, int out, void* stream)
{
    const int64_t total = a.M * a.N;
    const dim3 grid((unsigned)((total + 255) / 256)), block(256);
    if (act == VVH_F32 && out == VVH_F32) hipLaunchKernelGGL((k_generic<float, float>), grid, block, 0, S(stream), a);
    else if (act == VVH_F32) hipLaunchKernelGGL((k_generic<float, f16>), grid, block, 0, S(stream), a);
    else if (out == VVH_F32) hipLaunchKernelGGL((k_generic<f16, float>), grid, block, 0, S(stream), a);
    else hipLaunchKernelGGL((k_generic<f16, f16>), grid, block, 0, S(stream), a);
    return (int)hipGetLastError();
}

template <int MT>
static void gemv_f32_launch(const LinArgs& a, int out, dim3 grid, hipStream_t s)
{
    if (out == VVH_F32) hipLaunchKernelGGL((k_gemv_f32<MT, float>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_gemv_f32<MT, f16>), grid, dim3(256), 0, s, a);
}

int launch_gemv_f32(const LinArgs& a, int out, void* stream)
{
    const int64_t mt = a.M <= 1 ? 1 : a.M <= 2 ? 2 : a.M <= 4 ? 4 : 8;
    const dim3 grid((unsigned)decode_blocks(a), (unsigned)((a.M + mt - 1) / mt));
    switch (mt) {
        case 1: gemv_f32_launch<1>(a, out, grid, S(stream)); break;
        case 2: gemv_f32_launch<2>(a, out, grid, S(stream)); break;
        case 4: gemv_f32_launch<4>(a, out, grid, S(stream)); break;
        default: gemv_f32_launch<8>(a, out, grid, S(stream)); break;
    }
    return (int)hipGetLastError();
}

int launch_skinny(const LinArgs& a, int out, void* stream)
{
    const dim3 grid((unsigned)decode_blocks(a));
    if (out == VVH_F32) hipLaunchKernelGGL((k_skinny<float>), grid, dim3(256), 0, S(stream), a);
    else hipLaunchKernelGGL((k_skinny<f16>), grid, dim3(256), 0, S(stream), a);
    return (int)hipGetLastError();
}

int launch_skinny_grouped(const LinArgs* dev_table, int count, int64_t total_blocks, int out,
                          void* stream)
{
    const dim3 grid((unsigned)total_blocks);
    if (out == VVH_F32) hipLaunchKernelGGL((k_skinny_grouped<float>), grid, dim3(256), 0, S(stream), dev_table, count);
    else hipLaunchKernelGGL((k_skinny_grouped<f16>), grid, dim3(256), 0, S(stream), dev_table, count);
    return (int)hipGetLastError();
}

int launch_gemm(const LinArgs& a, int out, void* stream)
{
    const int64_t nbm = (a.M + kGemmBM - 1) / kGemmBM;
    const int64_t nbn = (a.N + kGemmBN - 1) / kGemmBN;
    const dim3 grid((unsigned)(nbm * nbn));
    if (out == VVH_F32) hipLaunchKernelGGL((k_gemm<float>), grid, dim3(256), 0, S(stream), a);
    else hipLaunchKernelGGL((k_gemm<f16>), grid, dim3(256), 0, S(stream), a);
    return (int)hipGetLastError();
}

}  // namespace vvh
