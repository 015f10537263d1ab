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

#include <algorithm>
#include <cstdlib>
#include <utility>

#include "common.h"
#include "device.h"

namespace vvh {

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

__device__ __forceinline__ u4 ld_stream_g(const int8_t* p)
{
    return __builtin_nontemporal_load(gbl(reinterpret_cast<const u4*>(p)));
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
    c.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: keeps the loops scalar
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
        acc[m] = sum_x32(sum_x16(acc[m]));
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
//
// Memory pipeline: the weight stream is the only HBM traffic, so each wave
// keeps two chunks of kDecodeDepth 16-byte loads per lane in flight (the
// next chunk is issued before the current one is consumed).  When the
// activations are small (M*K*2 <= kXLdsBytes) the block stages them once in
// LDS (rows padded by 16 bytes so the 16 rows of an MFMA operand fall in
// distinct banks); otherwise they are read through the L1/L2 caches.
// ---------------------------------------------------------------------------
constexpr int kDecodeDepth = 8;
constexpr int kXLdsBytes = 16384;
constexpr int kXLdsHalves = kXLdsBytes / 2 + 16 * 8;

struct DecodeShared {
    f4 red[4][64];
    __attribute__((aligned(16))) f16 xs[kXLdsHalves];
};

// at most kXLdsBytes of activations (the staging loop's 4 chunks per
// thread), in rows padded to K + 8 halves that fit xs (implied for M <= 16)
__device__ __forceinline__ bool decode_x_in_lds(const LinArgs& a)
{
    return a.M * a.K * 2 <= kXLdsBytes && a.M * (a.K + 8) <= kXLdsHalves;
}

// G > 1 (16 < M <= 16 G): the lane's activation rows are m, m + 16, ...,
// m + 16 (G - 1), one MFMA accumulator pair per group, so each weight chunk
// is loaded and converted once for all G groups.
template <typename OT, bool XLDS, int G = 1>
__device__ __forceinline__ void skinny_body(const LinArgs& a, int64_t block, DecodeShared& sh)
{
    constexpr int D = kDecodeDepth;
    const DecodeCoord c = decode_coord(a, block);
    const int64_t n0 = c.tile * kDecodeTileN;
    const int64_t nrow = n0 + (c.lane & 15) < a.N ? n0 + (c.lane & 15) : a.N - 1;
    const int chunk = c.lane >> 4;
    const int m = c.lane & 15;
    const bool active = n0 < a.N;
    const int8_t* wp = a.w + nrow * a.K + chunk * 16;
    const int64_t ldx = a.K + 8;  // padded LDS row stride of the staged activations
    const f16* xg = static_cast<const f16*>(a.inp);
    bool mvalid[G];
    const f16* xp[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int mg = m + 16 * g;
        mvalid[g] = mg < a.M;
        xp[g] = XLDS ? sh.xs + (mvalid[g] ? mg : 0) * ldx + chunk * 16 : xg + (mvalid[g] ? mg : 0) * a.K + chunk * 16;
    }

    u4 wa[D], wb[D];
    auto issue = [&](u4 (&buf)[D], int64_t s) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int64_t st = s + u;
            buf[u] = u4{0u, 0u, 0u, 0u};
            if (active && st < c.s1 && st * 64 + chunk * 16 < a.K) buf[u] = ld_stream(wp + st * 64);
        }
    };
    f4 acc0[G], acc1[G];
#pragma unroll
    for (int g = 0; g < G; g++) acc0[g] = acc1[g] = f4{0.f, 0.f, 0.f, 0.f};
    auto consume = [&](const u4 (&buf)[D], int64_t s) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int64_t st = s + u;
            if (st < c.s1) {
                h8 b0, b1;
                i8x16_to_h8x2(buf[u], b0, b1);
#pragma unroll
                for (int g = 0; g < G; g++) {
                    h8 xa = {}, xb = {};
                    if (mvalid[g] && st * 64 + chunk * 16 < a.K) {
                        xa = *reinterpret_cast<const h8*>(xp[g] + st * 64);
                        xb = *reinterpret_cast<const h8*>(xp[g] + st * 64 + 8);
                    }
                    acc0[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, b0, acc0[g], 0, 0, 0);
                    acc1[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xb, b1, acc1[g], 0, 0, 0);
                }
            }
        }
    };

    if (XLDS) {
        // activation loads first, then the first weight chunk, so both are in
        // flight while the activations are written to LDS
        constexpr int XL = kXLdsBytes / (256 * 16);
        const int64_t xchunks = a.M * a.K / 8;
        u4 xr[XL];
#pragma unroll
        for (int i = 0; i < XL; i++) {
            const int64_t idx = threadIdx.x + 256 * i;
            xr[i] = idx < xchunks ? *reinterpret_cast<const u4*>(xg + idx * 8) : u4{0u, 0u, 0u, 0u};
        }
        issue(wa, c.s0);
#pragma unroll
        for (int i = 0; i < XL; i++) {
            const int64_t idx = threadIdx.x + 256 * i;
            if (idx < xchunks) {
                const int64_t row = idx * 8 / a.K, col = idx * 8 - row * a.K;
                *reinterpret_cast<u4*>(sh.xs + row * ldx + col) = xr[i];
            }
        }
        // LDS writes done and visible to the block; the weight loads stay in flight
        lds_barrier();
    } else {
        issue(wa, c.s0);
    }

    if (active) {
        for (int64_t s = c.s0; s < c.s1; s += 2 * D) {
            issue(wb, s + D);
            consume(wa, s);
            if (s + 2 * D < c.s1) issue(wa, s + 2 * D);
            consume(wb, s + D);
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        f4 acc = acc0[g] + acc1[g];
        if (c.ksplit > 1) {
            if (g > 0) __syncthreads();  // the previous group's sums are read
            sh.red[c.wave][c.lane] = acc;
            __syncthreads();
            if (c.ks == 0) {
                for (int j = 1; j < c.ksplit; j++) acc += sh.red[c.wave + j][c.lane];
            }
        }
        if (c.ks == 0) {
            const int64_t n = n0 + (c.lane & 15);
            if (n < a.N) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int64_t mm = 16 * g + 4 * (c.lane >> 4) + r;
                    if (mm < a.M) store_out<OT>(a, mm, n, acc[r]);
                }
            }
        }
    }
}

template <typename OT, int G>
__global__ __launch_bounds__(256) void k_skinny(LinArgs a)
{
    __shared__ DecodeShared sh;
    if (decode_x_in_lds(a)) skinny_body<OT, true, G>(a, blockIdx.x, sh);
    else skinny_body<OT, false, G>(a, blockIdx.x, sh);
}

// Grouped launch: block b serves problem p with
// table[p].block_begin <= b < table[p+1].block_begin.
template <typename OT>
__global__ __launch_bounds__(256) void k_skinny_grouped(const LinArgs* __restrict__ table, int count)
{
    __shared__ DecodeShared sh;
    const int b = blockIdx.x;
    int lo = 0, hi = count - 1;
    while (lo < hi) {  // last p with block_begin <= b
        const int mid = (lo + hi + 1) >> 1;
        if (table[mid].block_begin <= b) lo = mid;
        else hi = mid - 1;
    }
    const LinArgs a = table[lo];
    if (decode_x_in_lds(a)) skinny_body<OT, true>(a, b - a.block_begin, sh);
    else skinny_body<OT, false>(a, b - a.block_begin, sh);
}

// ---------------------------------------------------------------------------
// k_dot: fp16 activations, M <= 16; dot products on VALU (M <= 2) or MFMA
// (M = 3..16, see MF below).
//
// The weight stream decides the speed of a decode GEMV, and it runs fastest
// when every load instruction covers whole 128-byte cache lines: 8 rows x
// 128 B per instruction streams about 7 TB/s on MI355X, the 16 rows x 64 B
// that a 16x16 MFMA operand needs about 5.5 TB/s.  So at M <= 16, where the
// MFMA's M side would be mostly empty anyway, each wave owns a 16-row tile
// and lane l reads the 16-byte chunk c = l%8 of the 128-byte k step of rows
// r = l/8 and r + 8 (two loads per step), converts the codes exactly to fp16
// and (M <= 2) accumulates v_dot2_f32_f16 products in fp32; with more rows
// the loaded tile is regathered through LDS into MFMA operands instead.  The 8 lanes of a row are
// summed with a butterfly at the end.  Activations are staged once per
// block in LDS (a broadcast read: the 8 rows of a wave read the same 8
// chunks), or read through the caches when they do not fit.
//
// Tiles and k steps are shared out as for k_skinny (decode_coord with
// 128-wide steps).  Every weight load is issued unconditionally (steps past
// the wave's range re-read its last step, chunks past K read inside the row)
// and masked when consumed, so the wait counts of the pipeline are fixed.
// ---------------------------------------------------------------------------
// The ring depth DEPTH (k steps of 2 loads each in flight per wave) is a
// template parameter, 2, 4 or 7, chosen per launch (dot_depth on the host)
// to hold the waves' k ranges where it can: each slot past a wave's range
// re-reads a step and costs issue time.

__device__ __forceinline__ DecodeCoord dot_coord(const LinArgs& a, int64_t block)
{
    DecodeCoord c;
    c.lane = threadIdx.x & 63;
    c.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: keeps the loops scalar
    c.ksplit = a.ksplit;  // 1, 2 or 4 (blocks of 4 waves), 8 (of 8): shifts, not divisions
    const int lg = __builtin_ctz(c.ksplit);
    c.ks = c.wave & (c.ksplit - 1);
    c.tile = block * ((c.ksplit > 4 ? 8 : 4) >> lg) + (c.wave >> lg);
    const int32_t steps = ((int32_t)a.K + kDotStep - 1) / kDotStep;  // K <= INT32_MAX - kDotStep
    const int32_t per = (steps + c.ksplit - 1) >> lg;
    c.s0 = c.ks * per < steps ? c.ks * per : steps;
    c.s1 = c.s0 + per < steps ? c.s0 + per : steps;
    return c;
}

// LDS of one k_dot block: the ksplit partial sums of the 16 rows of each
// wave, then (when they fit) the staged activations, M rows with a row
// stride of K + 8 halves.  The launcher sizes the dynamic LDS with the same
// rule (dot_lds_bytes), so kernel and launcher agree on where x lives.
template <int NW>
struct DotRedN {
    float v[NW][kDotMaxM][16];  // [wave][m][row]
};
using DotRed = DotRedN<4>;
static_assert(sizeof(DotRed) == kDotRedBytes, "reduction scratch size");

// 16 fp16 activations times 16 exact fp16 codes, accumulated in fp32.
__device__ __forceinline__ float dot16(const h8 w0, const h8 w1, const h8 x0, const h8 x1, float acc)
{
#pragma unroll
    for (int j = 0; j < 4; j++)
        acc = __builtin_amdgcn_fdot2(h2{w0[2 * j], w0[2 * j + 1]}, h2{x0[2 * j], x0[2 * j + 1]}, acc, false);
#pragma unroll
    for (int j = 0; j < 4; j++)
        acc = __builtin_amdgcn_fdot2(h2{w1[2 * j], w1[2 * j + 1]}, h2{x1[2 * j], x1[2 * j + 1]}, acc, false);
    return acc;
}

// Epilogue of one element through global-address-space pointers (the
// problem descriptor may come from a plan table, whose pointers the compiler
// would otherwise treat as generic and access with flat instructions).
// The decode epilogue acc * scale (+ bias) (+ residual) with the product
// rounded to fp32 before the additions (the empty asm keeps the compiler from
// fusing it into an FMA in one instantiation and not in another): both k_dot
// variants (operands loaded early or after the k loop) share it, so their
// outputs agree bit for bit.
__device__ __forceinline__ float dot_epi(float acc, float sc, bool has_bias, float bi, bool has_res, float res)
{
    float v = acc * sc;
    __asm__("" : "+v"(v));
    if (has_bias) v += bi;
    if (has_res) v += res;
    return v;
}

template <typename OT>
__device__ __forceinline__ void store_out_g(const LinArgs& a, int64_t m, int64_t n, float acc)
{
    const int64_t o = m * a.N + n;
    const float bi = a.bias ? *gbl(a.bias + n) : 0.0f;
    const float rv = a.res ? (float)*gbl(static_cast<const OT*>(a.res) + o) : 0.0f;
    *gbl(static_cast<OT*>(a.out) + o) = (OT)dot_epi(acc, *gbl(a.scales + n), a.bias != nullptr, bi, a.res != nullptr, rv);
}

// Epilogue of a q/k/v plan problem with RoPE (a.rope != 0) for the lane's
// rows A and B of each activation row m: the linear's value rounded to OT
// (what vvh_rope would read back), then for q/k rows the split-half rotation
// of the pair (rows A and B are i and i + D/2 of one head) at position
// pos + m, then the store; k and v rows also go to row pos + m of the cache.
// Bit-identical to the plan's plain store followed by vvh_rope_append.
// rc, rs: rope_cs of the pair at position pos + m (q and k rows).
template <typename OT, int MT, bool EARLY>
__device__ __forceinline__ void dot_store_rope(const LinArgs& a, int64_t pos, int64_t rowA, int64_t rowB,
                                               const float (&accA)[MT], const float (&accB)[MT],
                                               const float (&e_sc)[2], const float (&e_bi)[2], const OT (&e_res)[MT][2],
                                               const float (&rc)[MT], const float (&rs)[MT])
{
    const int64_t rows[2] = {rowA, rowB};
    float sc[2], bi[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        sc[h] = EARLY ? e_sc[h] : *gbl(a.scales + rows[h]);
        bi[h] = EARLY ? e_bi[h] : (a.bias ? *gbl(a.bias + rows[h]) : 0.0f);
    }
    OT* out = static_cast<OT*>(a.out);
    OT* cache = static_cast<OT*>(a.cache);
#pragma unroll
    for (int m = 0; m < MT; m++) {
        if (m >= a.M) continue;
        OT v[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t o = m * a.N + rows[h];
            const float rv = a.res ? (EARLY ? (float)e_res[m][h] : (float)*gbl(static_cast<const OT*>(a.res) + o))
                                   : 0.0f;
            v[h] = (OT)dot_epi(h ? accB[m] : accA[m], sc[h], a.bias != nullptr, bi[h], a.res != nullptr, rv);
        }
        if (a.rope != 3) {
            float r0, r1;
            rope_apply((float)v[0], (float)v[1], rc[m], rs[m], r0, r1);
            v[0] = (OT)r0;
            v[1] = (OT)r1;
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            *gbl(out + m * a.N + rows[h]) = v[h];
            if (a.rope != 1) *gbl(cache + (pos + m) * a.N + rows[h]) = v[h];
        }
    }
}

// SiLU-gated epilogue of a plan problem (a.glu): rows A and B of the lane
// are gate row i and up row N/2 + i; each linear value rounded to OT (what
// vvh_eltwise would read back), then silu(gate) * up, rounded once, to
// element i of output row m (rows of N / 2).  Bit-identical to the plan's
// plain store followed by vvh_eltwise(VVH_OP_SILU_MUL).
template <typename OT, int MT, bool EARLY>
__device__ __forceinline__ void dot_store_glu(const LinArgs& a, int64_t rowA, int64_t rowB,
                                              const float (&accA)[MT], const float (&accB)[MT],
                                              const float (&e_sc)[2], const float (&e_bi)[2])
{
    const int64_t rows[2] = {rowA, rowB};
    float sc[2], bi[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        sc[h] = EARLY ? e_sc[h] : *gbl(a.scales + rows[h]);
        bi[h] = EARLY ? e_bi[h] : (a.bias ? *gbl(a.bias + rows[h]) : 0.0f);
    }
    OT* out = static_cast<OT*>(a.out);
    const int64_t half = a.N / 2;
#pragma unroll
    for (int m = 0; m < MT; m++) {
        if (m >= a.M) continue;
        const OT g = (OT)dot_epi(accA[m], sc[0], a.bias != nullptr, bi[0], false, 0.0f);
        const OT u = (OT)dot_epi(accB[m], sc[1], a.bias != nullptr, bi[1], false, 0.0f);
        *gbl(out + m * half + rowA) = (OT)silu_mul_ref((float)g, (float)u);
    }
}

template <typename OT, int MT, int XS, bool EARLY, int DEPTH, int FS, int NW = 4>
__device__ __forceinline__ void dot_body(const LinArgs& a, int64_t block, char* smem, int64_t pos)
{
    // where the activations come from (XS, chosen per launch on the host):
    // kXLds staged once per block in LDS; kXDirect loaded with the weights,
    // as MFMA operands on the MF path; kXTile (MF only) loaded with the
    // weights in whole lines and regathered through the wave's LDS tile
    constexpr bool XLDS = XS == kXLds;
    constexpr bool XW = XS == kXTile;
    static_assert(!XW || MT >= 4, "the activation tile serves the MFMA path");
    // activations in the ring take 8 VGPRs per row and slot: halve the ring
    // for several rows so the wave keeps two waves per SIMD's worth of VGPRs,
    // except in early launches, whose few blocks occupancy does not bound
    // (graph-replayed, down projections at M = 2: 0.5B 7.35 -> 6.55 us, 1.5B
    // 10.32 -> 9.06 us with the whole ring)
    constexpr int D = (XLDS || MT == 1 || DEPTH < 4 || EARLY) ? DEPTH : DEPTH / 2;
    // MF (3-16 activation rows): the dot products on MFMA (16 rows x 16
    // columns, M of them used, 32 codes per instruction) instead of v_dot2:
    // the step's weights go through the wave's LDS tile into the MFMA
    // operand layout.  The activations (kXDirect) load as MFMA operands,
    // 16 rows x 64 B per instruction, which take the texture unit twice the
    // time per byte of whole-line loads; kXTile loads them in whole lines
    // (8 rows x 128 B, XI per step: rows 0-7, and 8-15 when MT = 16) and
    // regathers them through LDS as well, for launches whose tiles re-read
    // many activation bytes (the regathering adds latency to each step)
    constexpr bool MF = MT >= 4;
    constexpr int XI = XW ? (MT > 8 ? 4 : 2) : 4;
    // First stages (FS, chosen per launch by the host): the stage's operands
    // are requested before the weight ring and the stage runs while the
    // weights are in flight (the in-order wait counter lets a wait for them
    // leave the younger ring loads outstanding).
    //   kFirstRms / kFirstRms4: the RMSNorm stage of an early launch (xop 1,
    //     M <= 4, K <= 1024 / 2048): every wave loads the whole rows (chunks
    //     lane + 64 j, j < RJ) and sums their squares itself (rms_sumsq8,
    //     wave_sum_xor), then thread (w, l) normalizes chunk l + 64 w, which
    //     it holds; one barrier in all;
    //   kFirstAttn: the attention merge stage (xop 3, one row, K <= 1024);
    //   kFirstX1/3/5: one to four rows of plain activations (xop 0) in XR
    //     rounds of 256 chunks: loaded in the ring instead, each wave would
    //     request its activation chunks with every weight step, as many
    //     bytes per row as the weights through the texture unit.
    // A compile-time choice: chosen at run time, the other path's ring issue
    // comes before the stage's loads, and the compiler then waits for every
    // older load before the stage's first one (a whole round trip).
    constexpr int XR = FS == kFirstX1 ? 1 : FS == kFirstX3 ? 3 : FS == kFirstX5 ? 5 : 0;
    constexpr int RJ = FS == kFirstRms ? 2 : FS == kFirstRms4 ? 4 : 0;  // chunks of a row per lane
    constexpr bool rms_first = RJ > 0 && EARLY && XLDS && MT <= 4;
    constexpr bool attn_first = FS == kFirstAttn && EARLY && XLDS && MT == 1;
    constexpr bool x_first = XR > 0 && EARLY && XLDS && MT <= 4;
    constexpr bool first = rms_first || attn_first || x_first;
    static_assert(FS == kFirstNone || first, "a first stage this launch cannot run");
    // NW waves per block: 4, or 8 (k split 8) on the plain MFMA path with
    // the activations loaded with the weights; the reduction scratch and the
    // per-wave LDS tiles scale with it
    static_assert(NW == 4 || (NW == 8 && MT >= 4 && !XLDS && FS == kFirstNone), "8-wave blocks: plain MFMA path");
    constexpr int64_t RB = kDotRedBytes * NW / 4, WB = kDotWtBytes * NW / 4;
    DotRedN<NW>& red = *reinterpret_cast<DotRedN<NW>*>(smem);
    f16* xs = reinterpret_cast<f16*>(smem + RB);
    const DecodeCoord c = dot_coord(a, block);
    const int r = c.lane >> 3, ch = c.lane & 7;
    const int64_t n0 = c.tile * kDecodeTileN;
    const bool active = n0 < a.N && c.s0 < c.s1;
    // rows of the lane: n0 + r and n0 + 8 + r, or for rotated q/k rows the
    // pair (h*D + 8s + r, + D/2) of tile s of head h (rope_d % 16 == 0 and
    // N % rope_d == 0, checked when the plan gets its RoPE epilogue)
    const bool pair = a.rope == 1 || a.rope == 2;
    // an idle tile past the problem (the partly filled last block of a
    // launch) takes tile 0's rows, so its early loads of scales, biases,
    // residuals and weights stay inside the problem; it stores nothing
    const int64_t tile_r = n0 < a.N ? c.tile : 0;
    int64_t rowA, rowB;
    int32_t pidx = 0;  // rotated rows: the pair's index within its head, < rope_d / 2
    if (pair) {
        // 32-bit wave-uniform division (rows < 2^31, checked with the
        // epilogue, so tiles < 2^27): the rows feed the
        // first weight loads, so a 64-bit division here delays the whole ring
        const int32_t tph = a.rope_d >> 4;
        const int32_t t = __builtin_amdgcn_readfirstlane((int32_t)tile_r);
        const int32_t hd = t / tph, sd = t - hd * tph;
        pidx = 8 * sd + r;
        rowA = (int64_t)hd * a.rope_d + pidx;
        rowB = rowA + a.rope_d / 2;
    } else if (a.glu) {
        // gate row 8 t + r and its up row (N % 16 == 0: every tile is whole)
        rowA = tile_r * 8 + r;
        rowB = a.N / 2 + rowA;
    } else {
        rowA = n0 + r < a.N ? n0 + r : a.N - 1;
        rowB = n0 + 8 + r < a.N ? n0 + 8 + r : a.N - 1;
    }
    const int8_t* wpA = a.w + rowA * a.K;
    const int8_t* wpB = a.w + rowB * a.K;
    const int32_t kmax = (int32_t)a.K - 16;  // last valid chunk start of a row
    const int32_t s1 = (int32_t)c.s1;
    const int64_t ldx = a.K + 8;
    const f16* xg = static_cast<const f16*>(a.inp);
    // MF: lane l is MFMA row / column fi = l % 16 and k group fg = l / 16;
    // its activation row (clamped: columns past M are computed and unused)
    const int fi = c.lane & 15, fg = c.lane >> 4;
    const int32_t fm = fi < a.M ? fi : 0;
    char* wt = smem + RB + (XLDS ? a.M * ldx * 2 : 0) + c.wave * (16 * kDotWtPitch);
    char* xt = smem + RB + WB + c.wave * (16 * kDotXtPitch);  // XW

    // Ring of D slots, one k step each: the two weight chunks of the step
    // and, when the activations are not in LDS, their activation chunks
    // (loaded with the weights, so consuming a slot never waits on a younger
    // load).  Slot u is consumed, then refilled with the step D ahead.
    struct Slot {
        u4 w[2];
        h8 x[XLDS ? 1 : (MF ? XI : MT)][MF ? 1 : 2];  // MF: the step's 4 operand fragments or XI whole-line chunks
    };
    Slot ring[D];
    auto issue = [&](int u, int32_t st) {
        st = st < s1 ? st : s1 - 1;  // past the range: re-read the last step
        st = st > 0 ? st : 0;        // (never below step 0)
        int32_t k = st * kDotStep + ch * 16;
        k = k < kmax ? k : kmax;
        ring[u].w[0] = ld_stream_g(wpA + k);
        ring[u].w[1] = ld_stream_g(wpB + k);
        if (XW) {
            // chunk i: activation row 8 (i / 2) + r (clamped: rows past M
            // read row 0, computed and unused), values 64 (i % 2) + 8 ch ..
            // + 7 of the step (clamped into the row; masked when consumed)
#pragma unroll
            for (int i = 0; i < XI; i++) {
                const int xr = 8 * (i >> 1) + r;
                int32_t kx = st * kDotStep + 64 * (i & 1) + 8 * ch;
                kx = kx < (int32_t)a.K - 8 ? kx : (int32_t)a.K - 8;
                ring[u].x[i][0] = *gbl(reinterpret_cast<const h8*>(xg + (xr < a.M ? xr : 0) * a.K + kx));
            }
        } else if (!XLDS && MF) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                int32_t kx = st * kDotStep + 32 * j + 8 * fg;
                kx = kx < (int32_t)a.K - 8 ? kx : (int32_t)a.K - 8;
                ring[u].x[j][0] = *gbl(reinterpret_cast<const h8*>(xg + fm * a.K + kx));
            }
        } else if (!XLDS) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const f16* xp = xg + (m < a.M ? m : 0) * a.K + k;
                ring[u].x[m][0] = *gbl(reinterpret_cast<const h8*>(xp));
                ring[u].x[m][1] = *gbl(reinterpret_cast<const h8*>(xp + 8));
            }
        }
    };
    f4 facc = {0.0f, 0.0f, 0.0f, 0.0f};  // MF: rows 4 fg .. 4 fg + 3, column fi
    float accA[MT], accB[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) accA[m] = accB[m] = 0.0f;
    // No branches in here: a conditional read would split the slot into
    // basic blocks, the dot products would sink below the refills and the
    // ring would need a second register copy.  The activation read is
    // clamped into the row and masked instead.
    const h8 zero8 = {};
    auto consume = [&](int u, int32_t st) {
        if constexpr (MF) {
            // the wave's 16 rows x 128 codes: lane (r, ch) holds codes
            // 16 ch .. 16 ch + 15 of rows r and 8 + r; one wave's LDS
            // accesses complete in order, so the reads below see these
            // writes and the next step's writes follow these reads
            *reinterpret_cast<u4*>(wt + r * kDotWtPitch + 16 * ch) = ring[u].w[0];
            *reinterpret_cast<u4*>(wt + (8 + r) * kDotWtPitch + 16 * ch) = ring[u].w[1];
            if (XW) {
                // the step's activation rows, 128 values (256 B) each
#pragma unroll
                for (int i = 0; i < XI; i++)
                    *reinterpret_cast<h8*>(xt + (8 * (i >> 1) + r) * kDotXtPitch + 128 * (i & 1) + 16 * ch) =
                        ring[u].x[i][0];
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                // codes 32 j + 8 fg .. + 7 of row fi against the same k of activation row fi
                const int32_t kx = st * kDotStep + 32 * j + 8 * fg;
                typedef uint32_t u2v __attribute__((ext_vector_type(2)));
                const u2v cw = *reinterpret_cast<const u2v*>(wt + fi * kDotWtPitch + 32 * j + 8 * fg);
                const h8 af = i8x8_to_h8(cw[0], cw[1]);
                h8 bf;
                if (XLDS) {
                    const int32_t kc = kx < (int32_t)a.K - 8 ? kx : (int32_t)a.K - 8;
                    bf = *reinterpret_cast<const h8*>(xs + fm * ldx + kc);
                } else if (XW) {
                    // activation row fi of the tile (rows 0-7 only when MT <= 8)
                    const int xr = MT > 8 ? fi : (fi & 7);
                    bf = *reinterpret_cast<const h8*>(xt + xr * kDotXtPitch + 2 * (32 * j + 8 * fg));
                } else {
                    bf = ring[u].x[j][0];
                }
                bf = kx < (int32_t)a.K ? bf : zero8;  // past K: the clamped codes meet zeros
                facc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf, facc, 0, 0, 0);
            }
            return;
        }
        int32_t k = st * kDotStep + ch * 16;
        const bool kv = k < a.K;
        k = k < kmax ? k : kmax;
        h8 a0, a1, b0, b1;
        i8x16_to_h8x2(ring[u].w[0], a0, a1);
        i8x16_to_h8x2(ring[u].w[1], b0, b1);
#pragma unroll
        for (int m = 0; m < MT; m++) {
            h8 x0, x1;
            if (XLDS) {
                const int mr = m < a.M ? m : 0;
                x0 = *reinterpret_cast<const h8*>(xs + mr * ldx + k);
                x1 = *reinterpret_cast<const h8*>(xs + mr * ldx + k + 8);
            } else {
                x0 = ring[u].x[m][0];
                x1 = ring[u].x[m][1];
            }
            const bool xv = kv && m < a.M;
            x0 = xv ? x0 : zero8;
            x1 = xv ? x1 : zero8;
            accA[m] = dot16(a0, a1, x0, x1, accA[m]);
            accB[m] = dot16(b0, b1, x0, x1, accB[m]);
        }
    };

    // EARLY (launches with few blocks, where latency and not occupancy sets
    // the time): the epilogue operands of the lane's two rows and the weight
    // ring are requested first, so the activation staging below waits for
    // them together instead of one after the other, and nothing is loaded
    // after the k loop.  Otherwise the ring is issued after the staging:
    // issued before it, the ring's 64 VGPRs stay live through the staging
    // and occupancy drops from 5 to 3 waves per SIMD (measured 5.9 -> 5.3
    // TB/s on the grouped decode set).
    float e_sc[2] = {0.0f, 0.0f}, e_bi[2] = {0.0f, 0.0f};
    OT e_res[MT][2];
    // MF, plain epilogue: the operands of the lane's outputs in the MFMA
    // tile's own layout, activation row fi and columns n0 + 4 fg + q
    float f_sc[4], f_bi[4];
    OT f_res[4];
    // RoPE cosine and sine of the lane's pair for each activation row (q and
    // k rows).  Early launches work them out right after requesting the
    // weights, while the loads are in flight: they take a long chain of fp64
    // operations that depends only on the position and the pair.
    // Positions the plan's cosine/sine table holds (every row's, tab) are
    // read from it with the other epilogue operands and only used at the
    // store; past the table they come from the pair's frequency.  Either
    // way the values are rope_cs_freq's, so the table changes no bit.
    float rc[MT], rs[MT], rfreq = 0.0f;
    f2 rt[MT];
    const bool tab = pos >= 0 && pos + a.M <= a.rope_cs_n;
    auto rope_load = [&]() {
        if (pair) {
            rfreq = *gbl(a.rope_freq + pidx);
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const int64_t pm = pos + m < a.rope_cs_n ? pos + m : a.rope_cs_n - 1;
                rt[m] = *gbl(reinterpret_cast<const f2*>(a.rope_cs) + pm * (a.rope_d / 2) + pidx);
            }
        }
    };
    auto rope_prep = [&]() {
        if (pair && !tab) {
#pragma unroll
            for (int m = 0; m < MT; m++) rope_cs_freq(pos + m, rfreq, rc[m], rs[m]);
        }
    };
    // the epilogue operands of an early launch (unconditional loads: an
    // absent bias or residual reads the scales, unused); the attention merge
    // stage requests them after the weight ring, behind its 16 part loads per
    // thread (o + merge 3.67 -> 3.53 us graph-replayed); the other stages
    // before their loads, where after the ring they measured slower (down
    // 4.56 -> 4.95 us)
    auto epi_load = [&]() {
        const float* bp = a.bias ? a.bias : a.scales;
        const OT* rp = a.res ? static_cast<const OT*>(a.res) : reinterpret_cast<const OT*>(a.scales);
        if constexpr (MF) {
            // clamped into the problem: columns past N and rows past M are
            // read again and not stored
            const int64_t mo = a.res ? (int64_t)(fi < a.M ? fi : 0) * a.N : 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int64_t n = n0 + 4 * fg + q < a.N ? n0 + 4 * fg + q : a.N - 1;
                f_sc[q] = *gbl(a.scales + n);
                f_bi[q] = *gbl(bp + n);
                f_res[q] = *gbl(rp + mo + n);
            }
        } else {
            const int64_t rows[2] = {rowA, rowB};
#pragma unroll
            for (int h = 0; h < 2; h++) {
                e_sc[h] = *gbl(a.scales + rows[h]);
                e_bi[h] = *gbl(bp + rows[h]);
#pragma unroll
                for (int m = 0; m < MT; m++) e_res[m][h] = *gbl(rp + (a.res && m < a.M ? m * a.N : 0) + rows[h]);
            }
        }
    };
    if constexpr (EARLY) {
        if constexpr (!attn_first) epi_load();
        rope_load();
        if constexpr (!first) {
            if (active) {
#pragma unroll
                for (int u = 0; u < D; u++) issue(u, (int32_t)c.s0 + u);
            }
            rope_prep();
        }
    }
    if constexpr (first) {
        if constexpr (rms_first) {
            // lane l: chunks l + 64 j of every row (clamped into the row past
            // its end: those add an exact 0), and the norm weights of its own
            // chunk l + 64 w
            const int32_t kc = (int32_t)(a.K / 8), co = c.lane + 64 * c.wave;
            const int32_t cw = co < kc ? co : kc - 1;
            h8 xv[MT][RJ > 0 ? RJ : 1];
#pragma unroll
            for (int j = 0; j < RJ; j++) {
                const int32_t ci = c.lane + 64 * j < kc ? c.lane + 64 * j : kc - 1;
#pragma unroll
                for (int m = 0; m < MT; m++)
                    xv[m][j] = *gbl(reinterpret_cast<const h8*>(xg + (m < a.M ? m : 0) * a.K + 8 * ci));
            }
            const f4 w0 = *gbl(reinterpret_cast<const f4*>(a.xw + 8 * cw));
            const f4 w1 = *gbl(reinterpret_cast<const f4*>(a.xw + 8 * cw + 4));
            // keep every row load ahead of the ring in issue order, and issue the
            // ring in every wave (an inactive wave's slots read clamped, in-bounds
            // rows and steps, unused): a wait for a row value then always counts
            // exactly the ring's loads as younger
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < D; u++) issue(u, (int32_t)c.s0 + u);
            __builtin_amdgcn_sched_barrier(0);
            rope_prep();
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m < a.M) {
                    float ss = 0.0f;
                    h8 own = xv[m][0];
#pragma unroll
                    for (int j = 0; j < RJ; j++) {
                        ss = rms_sumsq_h8(ss, xv[m][j], c.lane + 64 * j < kc);
                        own = j == c.wave ? xv[m][j] : own;
                    }
                    const float rv = rms_of(wave_sum_xor(ss), a.K, a.xeps);
                    if (co < kc) {
                        h8 v;
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            v[e] = (f16)rms_apply((float)own[e], rv, w0[e]);
                            v[4 + e] = (f16)rms_apply((float)own[4 + e], rv, w1[e]);
                        }
                        *reinterpret_cast<h8*>(xs + m * ldx + 8 * co) = v;
                    }
                }
            }
            __syncthreads();
        } else if constexpr (attn_first) {
            // element e = h hd + d of the row: the parts of head h merged in
            // part order (what k_attention_decode_mfma does with its waves);
            // thread t takes elements 4t .. 4t + 3 (K <= 1024).  No branch
            // around the loads (a conditional load would make the compiler
            // wait for every older one): slots past the part count re-read
            // part np - 1 and threads past K / 4 the last chunk, unused
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            const float* pp = static_cast<const float*>(a.inp);
            // xhd is a power of two (checked by vvh_linear_q8_dev_attn): shifts
            // instead of divisions ahead of the part loads
            const int32_t hd = a.xhd, lg = __builtin_ctz((uint32_t)hd), np = a.xparts, pitch = hd + 4;
            const int32_t heads = (int32_t)a.K >> lg, chunks = (int32_t)a.K / 4;
            const int32_t idx0 = (int32_t)threadIdx.x, idx = idx0 < chunks ? idx0 : chunks - 1;
            const int32_t e0 = 4 * idx, h = e0 >> lg, d0 = e0 & (hd - 1);
            f4 po[kAttnMaxParts];
            f2 pml[kAttnMaxParts];
#pragma unroll
            for (int pc = 0; pc < kAttnMaxParts; pc++) {
                const int32_t pcc = pc < np ? pc : np - 1;
                const float* pr = pp + ((int64_t)pcc * heads + h) * pitch;
                po[pc] = *gbl(reinterpret_cast<const f4*>(pr + d0));
                pml[pc] = *gbl(reinterpret_cast<const f2*>(pr + hd));
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < D; u++) issue(u, (int32_t)c.s0 + u);
            epi_load();
            __builtin_amdgcn_sched_barrier(0);
            if (idx0 < chunks) {
                // slots past np hold part np - 1 again: the maximum is the
                // same, and their sums are computed and dropped by a select
                // (no branch per part, and no 0 * inf where a part holds inf)
                float M = -INFINITY;
#pragma unroll
                for (int pc = 0; pc < kAttnMaxParts; pc++) M = fmaxf(M, pml[pc][0]);
                float num[4] = {0.0f, 0.0f, 0.0f, 0.0f}, den = 0.0f;
#pragma unroll
                for (int pc = 0; pc < kAttnMaxParts; pc++) {
                    const bool live = pc < np;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float nj = num[j], dj = den;
                        attn_merge_add(nj, dj, pml[pc][0], M, po[pc][j], pml[pc][1]);
                        num[j] = live ? nj : num[j];
                        if (j == 0) den = live ? dj : den;
                    }
                }
                const h4 v = {(f16)(num[0] / den), (f16)(num[1] / den), (f16)(num[2] / den), (f16)(num[3] / den)};
                *reinterpret_cast<h4*>(xs + e0) = v;
            }
            __syncthreads();
        } else if constexpr (x_first) {
            // chunk i of the rows (row i / (K / 8)): round i / 256 of thread
            // i % 256; the loads of the rounds past the rows re-read the last
            // chunk, unused
            const int32_t rchunks = (int32_t)(a.K / 8), xchunks = (int32_t)a.M * rchunks;
            h8 xr[XR > 0 ? XR : 1];
#pragma unroll
            for (int i = 0; i < XR; i++) {
                int32_t idx = (int32_t)threadIdx.x + 256 * i;
                idx = idx < xchunks ? idx : xchunks - 1;
                xr[i] = *gbl(reinterpret_cast<const h8*>(xg + 8 * idx));  // rows are contiguous in the input
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < D; u++) issue(u, (int32_t)c.s0 + u);
            __builtin_amdgcn_sched_barrier(0);
            rope_prep();
#pragma unroll
            for (int i = 0; i < XR; i++) {
                const int32_t idx = (int32_t)threadIdx.x + 256 * i;
                int32_t m = 0;  // LDS rows of K + 8 halves
#pragma unroll
                for (int q = 1; q < MT; q++) m += idx >= q * rchunks ? 1 : 0;
                if (idx < xchunks) *reinterpret_cast<h8*>(xs + m * ldx + 8 * (idx - m * rchunks)) = xr[i];
            }
            __syncthreads();
        }
    }
    if constexpr (XLDS && !first) {
        // activations to LDS (through the input stage a.xop), 4 chunks of 8
        // values per thread per round; a round's loads are clamped into the
        // input and its stores masked, so all of them are in flight at once
        const int xop = a.xop;
        const int32_t K32 = (int32_t)a.K, xchunks = (int32_t)(a.M * a.K / 8);
        const int64_t ldin = xop == 2 ? 2 * a.K : a.K;  // [gate | up] rows for SiLU-mul
        float rinv[MT];                                 // RMSNorm divisor of each row
#pragma unroll
        for (int m = 0; m < MT; m++) rinv[m] = 1.0f;
        if (xop == 1) {
            // per row as k_rms_norm (every wave sums the whole row itself)
#pragma unroll
            for (int m = 0; m < MT; m++) {
                if (m < a.M) {
                    const f16* xr = xg + m * a.K;
                    float ss = 0.0f;
                    for (int32_t ci = c.lane; 8 * ci < K32; ci += 64)
                        ss = rms_sumsq_h8(ss, *gbl(reinterpret_cast<const h8*>(xr + 8 * ci)), true);
                    rinv[m] = rms_of(wave_sum_xor(ss), a.K, a.xeps);
                }
            }
        }
        constexpr int XL = 4;
        for (int32_t base = 0; base < xchunks; base += 256 * XL) {
            h8 xr[XL], yr[XL];
#pragma unroll
            for (int i = 0; i < XL; i++) {
                int32_t idx = base + (int32_t)threadIdx.x + 256 * i;
                idx = idx < xchunks ? idx : xchunks - 1;
                const int32_t row = idx * 8 / K32, col = idx * 8 - row * K32;
                const f16* p = xg + row * ldin + col;
                xr[i] = *gbl(reinterpret_cast<const h8*>(p));
                if (xop == 2) yr[i] = *gbl(reinterpret_cast<const h8*>(p + a.K));
            }
#pragma unroll
            for (int i = 0; i < XL; i++) {
                const int32_t idx = base + (int32_t)threadIdx.x + 256 * i;
                if (idx >= xchunks) continue;
                const int32_t row = idx * 8 / K32, col = idx * 8 - row * K32;
                h8 v = xr[i];
                if (xop == 1) {
                    float rv = rinv[0];
#pragma unroll
                    for (int m = 1; m < MT; m++) rv = row == m ? rinv[m] : rv;
                    const f4 w0 = *gbl(reinterpret_cast<const f4*>(a.xw + col));
                    const f4 w1 = *gbl(reinterpret_cast<const f4*>(a.xw + col + 4));
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        v[j] = (f16)rms_apply((float)xr[i][j], rv, w0[j]);
                        v[4 + j] = (f16)rms_apply((float)xr[i][4 + j], rv, w1[j]);
                    }
                } else if (xop == 2) {
#pragma unroll
                    for (int j = 0; j < 8; j++) v[j] = (f16)silu_mul_ref((float)xr[i][j], (float)yr[i][j]);
                }
                *reinterpret_cast<h8*>(xs + row * ldx + col) = v;
            }
        }
        __syncthreads();
    }

    int32_t s = (int32_t)c.s0;
    if (active) {
        if constexpr (!EARLY) {
#pragma unroll
            for (int u = 0; u < D; u++) issue(u, s + u);
        }
        // while steps remain beyond the ring: consume slot u, refill it with
        // the step D ahead (a refill past the range re-reads the last step,
        // so every wait in the loop counts the same D - 1 steps of loads)
        // (the scheduling barrier keeps each refill below the last read of
        // its slot: hoisted above it, the refill would land in other
        // registers that must be copied back at the loop edge, and those
        // copies wait for every outstanding load)
        for (; s + D < s1; s += D) {
#pragma unroll
            for (int u = 0; u < D; u++) {
                consume(u, s + u);
                __builtin_amdgcn_sched_barrier(0);
                issue(u, s + u + D);
            }
        }
        // the ring holds the last steps s .. s1 - 1 (at most D)
#pragma unroll
        for (int u = 0; u < D; u++) {
            if (s + u < s1) consume(u, s + u);
        }
    }
    if constexpr (MF) {
        // the MFMA tile (rows 4 fg + q of column fi) into the reduction
        // scratch, the ksplit waves of its tile added in wave order
        if (fi < MT) {
#pragma unroll
            for (int q = 0; q < 4; q++) red.v[c.wave][fi][4 * fg + q] = facc[q];
        }
        __syncthreads();
        const int w0 = c.ks == 0 ? c.wave : c.wave - c.ks;
        if (!a.glu && a.rope == 0) {
            // plain epilogue in the MFMA layout: lane (fi, fg) of the tile's
            // first wave stores activation row fi, columns n0 + 4 fg + q (the
            // same sums in the same order as the row layout below; 4 stores
            // per lane instead of 2 M per lane of one lane in eight)
            if (c.ks == 0 && fi < a.M && n0 < a.N) {
                if constexpr (!EARLY) epi_load();
                float s4[4];
#pragma unroll
                for (int q = 0; q < 4; q++) s4[q] = red.v[w0][fi][4 * fg + q];
                for (int j = 1; j < c.ksplit; j++) {
#pragma unroll
                    for (int q = 0; q < 4; q++) s4[q] += red.v[w0 + j][fi][4 * fg + q];
                }
                OT* out = static_cast<OT*>(a.out) + fi * a.N;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int64_t n = n0 + 4 * fg + q;
                    if (n < a.N)
                        *gbl(out + n) = (OT)dot_epi(s4[q], f_sc[q], a.bias != nullptr, f_bi[q], a.res != nullptr,
                                                    (float)f_res[q]);
                }
            }
            return;
        }
        // SiLU-gated and RoPE epilogues: every lane takes its rows r and 8 + r
#pragma unroll
        for (int m = 0; m < MT; m++) {
            accA[m] = red.v[w0][m][r];
            accB[m] = red.v[w0][m][8 + r];
        }
        for (int j = 1; j < c.ksplit; j++) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                accA[m] += red.v[w0 + j][m][r];
                accB[m] += red.v[w0 + j][m][8 + r];
            }
        }
    }
    // sum the 8 chunk lanes of each row (DPP steps: lanes 1, 2, then 4 apart)
    if constexpr (!MF) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            accA[m] = group_sum(accA[m], 8);
            accB[m] = group_sum(accB[m], 8);
        }
    }
    if (!MF && c.ksplit > 1) {
        if (ch == 0) {
#pragma unroll
            for (int m = 0; m < MT; m++) {
                red.v[c.wave][m][r] = accA[m];
                red.v[c.wave][m][8 + r] = accB[m];
            }
        }
        __syncthreads();
        if (c.ks == 0) {
            for (int j = 1; j < c.ksplit; j++) {
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    accA[m] += red.v[c.wave + j][m][r];
                    accB[m] += red.v[c.wave + j][m][8 + r];
                }
            }
        }
    }
    // (with MF these load their operands here: the early loads took the
    // plain epilogue's layout)
    if (a.glu) {
        if (c.ks == 0 && ch == 0 && n0 < a.N)
            dot_store_glu<OT, MT, EARLY && !MF>(a, rowA, rowB, accA, accB, e_sc, e_bi);
        return;
    }
    if (a.rope != 0) {
        if (c.ks == 0 && ch == 0 && n0 < a.N) {
            if constexpr (!EARLY) {
                rope_load();
                rope_prep();
            }
            if (tab) {
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    rc[m] = rt[m][0];
                    rs[m] = rt[m][1];
                }
            }
            dot_store_rope<OT, MT, EARLY && !MF>(a, pos, rowA, rowB, accA, accB, e_sc, e_bi, e_res, rc, rs);
        }
        return;
    }
    if constexpr (MF) return;  // (the plain epilogue took the MFMA layout above)
    if (c.ks == 0 && ch == 0 && n0 < a.N) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            if (m < a.M) {
                if constexpr (EARLY) {
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const int64_t n = n0 + 8 * h + r;
                        if (n < a.N)
                            *gbl(static_cast<OT*>(a.out) + m * a.N + n) =
                                (OT)dot_epi(h ? accB[m] : accA[m], e_sc[h], a.bias != nullptr, e_bi[h],
                                            a.res != nullptr, (float)e_res[m][h]);
                    }
                } else {
                    if (n0 + r < a.N) store_out_g<OT>(a, m, n0 + r, accA[m]);
                    if (n0 + 8 + r < a.N) store_out_g<OT>(a, m, n0 + 8 + r, accB[m]);
                }
            }
        }
    }
}

// XS = the activations' source (kXLds: staged in LDS, dot_x_in_lds, decided
// on the host for the launch: for a grouped launch it must hold for every
// problem; kXDirect, kXTile: loaded with the weights).
// The fields that the first loads of a block depend on come first, as scalar
// arguments, which arrive preloaded into registers at dispatch (14 dwords
// here; the struct is read from the kernel-argument segment when used).
// mk = M | ksplit << 8; xi = xparts | xhd << 8 for the attention merge stage
// (its part loads need both), else 0.
// A plain call has no RoPE or SiLU-gated epilogue.
template <typename OT, int MT, int XS, bool EARLY, int DEPTH, int FS, int NW>
__global__ __launch_bounds__(64 * NW) void k_dot(const int8_t* w, const void* inp, const float* scales,
                                             const float* bias, const void* res, int32_t N, int32_t K, int32_t mk,
                                             int32_t xi, const LinArgs a)
{
    extern __shared__ __attribute__((aligned(16))) char dot_smem[];
    LinArgs b = a;
    b.w = w;
    b.inp = inp;
    b.scales = scales;
    b.bias = bias;
    b.res = res;
    b.N = N;
    b.M = mk & 0xff;
    b.K = K;
    b.ksplit = mk >> 8;
    if constexpr (FS == kFirstAttn) {
        b.xparts = xi & 0xff;
        b.xhd = xi >> 8;
    }
    b.rope = 0;
    b.glu = 0;
    dot_body<OT, MT, XS, EARLY, DEPTH, FS, NW>(b, blockIdx.x, dot_smem, 0);
}

// Grouped launch.  count <= kDotInline: the problems are g.p[0, count) and
// b1, b2, b3 are the first blocks of problems 1, 2, 3 (INT32_MAX where there
// is none), all in the kernel arguments, so the block's problem is found
// without a memory load (the leading scalar arguments are preloaded into
// registers at dispatch); larger plans: block b serves problem
// table[block_prob[b]].  `pos`: the position of activation row 0 for
// problems with a RoPE epilogue.
//
// EP: the epilogue kinds the launch's problems use, fixed per launch by the
// host where it pays (single-row plans of the decode step): kEpiAny keeps
// every epilogue behind a run-time test; kEpiPlain, kEpiGlu and kEpiRope
// compile in one kind only.  The code of an epilogue a kernel can take but
// does not run still cost a one-row plan about 0.3 us per launch
// (graph-replayed, a 9728 x 896 plan: 4.68 against 4.37 us).
template <typename OT, int MT, int XS, bool EARLY, int DEPTH, int FS, int EP>
__global__ __launch_bounds__(256) void k_dot_grouped(int32_t b1, int32_t b2, int32_t b3, int32_t count, int64_t pos,
                                                     const LinArgs* __restrict__ table,
                                                     const int32_t* __restrict__ block_prob, const DotGroup g)
{
    extern __shared__ __attribute__((aligned(16))) char dot_smem[];
    const int b = blockIdx.x;
    LinArgs a;
    if (count <= kDotInline) a = g.p[(b >= b1) + (b >= b2) + (b >= b3)];
    else a = table[*cst(block_prob + b)];
    if constexpr (EP == kEpiPlain) {
        a.rope = 0;
        a.glu = 0;
    } else if constexpr (EP == kEpiGlu) {
        a.rope = 0;
        a.glu = 1;
    } else if constexpr (EP == kEpiRope) {
        a.glu = 0;
    }
    dot_body<OT, MT, XS, EARLY, DEPTH, FS>(a, b - a.block_begin, dot_smem, pos);
}

// ---------------------------------------------------------------------------
// k_stream: persistent streaming decode, fp16 activations, M <= 16.
//
// Same per-step arithmetic as k_skinny (a 16-row tile, lane l streams 16
// codes of row n0 + l%16 at k = 64s + 16(l/16), two v_mfma_f32_16x16x32_f16
// per 64-wide step), but the work is organised for the HBM stream:
//   - each wave is independent (no LDS, no barriers) and walks a list of
//     tiles (StreamArgs), so a launch is about 8 resident waves per CU that
//     each stream a long run of weights;
//   - a ring of D register slots keeps D 16-byte weight loads per lane in
//     flight at all times, across tile boundaries: slot u is consumed, then
//     refilled with the step D positions ahead, which may belong to the
//     next tile;
//   - the activation fragment of a step is loaded into the same slot as its
//     weights (lanes whose row m >= M load nothing), and the epilogue
//     operands of a tile (scale, bias, residual) are loaded when the issue
//     side enters the tile, so no load is ever waited on before the loads
//     issued ahead of it have landed anyway.
// Every problem has nsteps = ceil(K/64) >= D, so the issue side is at most
// one tile ahead of the consume side: two tile descriptors suffice.
// ---------------------------------------------------------------------------
struct StreamTile {
    const int8_t* w;
    const f16* x;
    const float* sc;
    const float* bi;
    const void* res;
    void* out;
    int64_t M, N, K, n0;
    int32_t nsteps;
};

template <bool ONE>
__device__ __forceinline__ void stream_tile(const StreamArgs& sa, int64_t g, StreamTile& t)
{
    LinArgs A;
    int64_t lt;
    if (ONE) {
        A = sa.one;
        lt = g;
    } else {
        const int p = *cst(sa.tile_prob + g);
        const VVH_CONST LinArgs* ap = cst(sa.table) + p;
        A.w = ap->w;
        A.inp = ap->inp;
        A.scales = ap->scales;
        A.bias = ap->bias;
        A.res = ap->res;
        A.out = ap->out;
        A.M = ap->M;
        A.N = ap->N;
        A.K = ap->K;
        lt = g - ap->tile_begin;
    }
    t.w = A.w;
    t.x = static_cast<const f16*>(A.inp);
    t.sc = A.scales;
    t.bi = A.bias;
    t.res = A.res;
    t.out = A.out;
    t.M = A.M;
    t.N = A.N;
    t.K = A.K;
    t.n0 = lt * kDecodeTileN;
    t.nsteps = (int32_t)((A.K + 63) / 64);
}

// Epilogue operands of one step for this lane (channel n0 + l%16, rows
// 4(l/16) + r, r < MR), loaded in the same ring slot as the step's weights
// and kept as loaded (converting a residual right after its load would wait
// on it).  Only the last step of a tile uses them, but loading them for every
// step keeps the number of vector memory operations per slot fixed: every
// static s_waitcnt in the loop then counts about D slots of loads, whatever
// path the wave takes at tile boundaries.  Every load reads an in-bounds
// address (channel clamped to N-1, row to 0, absent bias or residual read
// from the scales) and is masked in the epilogue.
template <typename OT, int MR>
struct StreamEpi {
    float sc, bi;
    OT res[MR];
};

template <typename OT, int MR>
__device__ __forceinline__ void stream_epi_store(const StreamTile& t, int lane, const StreamEpi<OT, MR>& e, f4 acc)
{
    const int64_t n = t.n0 + (lane & 15);
    if (n >= t.N) return;
    const float bi = t.bi ? e.bi : 0.0f;
#pragma unroll
    for (int r = 0; r < MR; r++) {
        const int64_t m = 4 * (lane >> 4) + r;
        if (m < t.M) {
            const float rv = t.res ? (float)e.res[r] : 0.0f;
            *gbl(static_cast<OT*>(t.out) + m * t.N + n) = (OT)(acc[r] * e.sc + bi + rv);
        }
    }
}

// MR = residual rows per lane: 1 when every problem has M == 1 (only lanes
// 0-15 hold a valid row), else 4.
template <typename OT, int D, bool ONE, int MR>
__global__ __launch_bounds__(256, 2) void k_stream(const StreamArgs sa)
{
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * 256u + threadIdx.x) >> 6));
    if (wave >= sa.waves) return;
    const int r16 = lane & 15, chunk = lane >> 4;

    int64_t pos, end;
    if (sa.mode == kStreamRange) {
        pos = sa.total_tiles * wave / sa.waves;
        end = sa.total_tiles * (wave + 1) / sa.waves;
    } else {
        pos = *cst(sa.list_off + wave);
        end = *cst(sa.list_off + wave + 1);
    }
    auto next_tile = [&]() -> int64_t {
        if (pos >= end) return -1;
        const int64_t g = sa.mode == kStreamRange ? pos : (int64_t)*cst(sa.list + pos);
        pos++;
        return g;
    };

    u4 sw[D];
    h8 sxa[D], sxb[D];
    StreamEpi<OT, MR> se[D];
    // per-lane issue pointers of the issue tile; the chunk offset is clamped
    // so that the k tail of a K % 64 != 0 row still reads inside the row
    const int8_t* iwp;
    const f16* ixp;
    const float *iscp, *ibip;
    const OT* irp[MR];
    int64_t ikmax;  // last valid 16-element chunk start of a row
    auto issue_setup = [&](const StreamTile& t) {
        const int64_t nc = t.n0 + r16 < t.N ? t.n0 + r16 : t.N - 1;
        iwp = t.w + nc * t.K;
        ixp = t.x + (r16 < t.M ? r16 : 0) * t.K;
        ikmax = t.K - 16;
        iscp = t.sc + nc;
        ibip = (t.bi ? t.bi : t.sc) + nc;
#pragma unroll
        for (int r = 0; r < MR; r++) {
            const int64_t m = 4 * chunk + r;
            irp[r] = t.res ? static_cast<const OT*>(t.res) + (m < t.M ? m : 0) * t.N + nc
                           : reinterpret_cast<const OT*>(t.sc);
        }
    };
    auto issue = [&](int u, int64_t s) {
        int64_t k = s * 64 + chunk * 16;
        k = k < ikmax ? k : ikmax;
        sw[u] = ld_stream_g(iwp + k);
        sxa[u] = *gbl(reinterpret_cast<const h8*>(ixp + k));
        sxb[u] = *gbl(reinterpret_cast<const h8*>(ixp + k + 8));
        se[u].sc = *gbl(iscp);
        se[u].bi = *gbl(ibip);
#pragma unroll
        for (int r = 0; r < MR; r++) se[u].res[r] = *gbl(irp[r]);
    };

    StreamTile cT, iT;
    bool has_n = false;   // the issue side is in the tile after cT
    bool idone = false;   // no tile left: the issue side re-reads its last step
    int32_t cs = 0, is = 0;

    const int64_t g0 = next_tile();
    if (g0 < 0) return;
    stream_tile<ONE>(sa, g0, cT);
    iT = cT;
    issue_setup(iT);

    auto advance_issue = [&]() {
        const int64_t g = next_tile();
        if (g < 0) {
            idone = true;
            is = iT.nsteps - 1;
            return;
        }
        stream_tile<ONE>(sa, g, iT);
        issue_setup(iT);
        has_n = true;
        is = 0;
    };

#pragma unroll
    for (int u = 0; u < D; u++) issue(u, is++);
    if (is == iT.nsteps) advance_issue();

    f4 acc0 = {0.f, 0.f, 0.f, 0.f};
    f4 acc1 = {0.f, 0.f, 0.f, 0.f};
    const h8 zero8 = {};
    for (;;) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            {
                // rows m >= M and the k tail beyond K contribute zero
                const bool xv = r16 < cT.M && (int64_t)cs * 64 + chunk * 16 < cT.K;
                h8 b0, b1;
                i8x16_to_h8x2(sw[u], b0, b1);
                acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv ? sxa[u] : zero8, b0, acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(xv ? sxb[u] : zero8, b1, acc1, 0, 0, 0);
            }
            if (++cs == cT.nsteps) {
                stream_epi_store<OT, MR>(cT, lane, se[u], acc0 + acc1);
                if (!has_n) return;
                cT = iT;
                has_n = false;
                cs = 0;
                acc0 = f4{0.f, 0.f, 0.f, 0.f};
                acc1 = f4{0.f, 0.f, 0.f, 0.f};
            }
            issue(u, is);
            if (!idone && ++is == iT.nsteps) advance_issue();
        }
    }
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
// k_splitk_reduce: out = (sum over splits of ws[s][m][n]) * scale[n] + bias[n]
// (+ res[m][n]), in fp32 with one rounding; 4 consecutive outputs per thread
// (16-byte partial loads when N % 4 == 0).  The partials are summed in split
// order, so the result does not depend on the launch.
// ---------------------------------------------------------------------------
template <typename OT>
__global__ __launch_bounds__(256) void k_splitk_reduce(LinArgs a)
{
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_row = (a.N + 3) / 4;
    if (q >= a.M * per_row) return;
    const int64_t m = q / per_row, n = (q - m * per_row) * 4;
    const int64_t o = m * a.N + n, plane = a.M * a.N;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.N % 4 == 0) {
        // four splits' loads in flight before their sums
        int32_t s = 0;
        for (; s + 4 <= a.nsplit; s += 4) {
            f4 p[4];
#pragma unroll
            for (int j = 0; j < 4; j++) p[j] = *reinterpret_cast<const f4*>(a.ws + (s + j) * plane + o);
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] += p[j][e];
        }
        for (; s < a.nsplit; s++) {
            const f4 p = *reinterpret_cast<const f4*>(a.ws + s * plane + o);
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] += p[e];
        }
    } else {
        for (int32_t s = 0; s < a.nsplit; s++)
            for (int e = 0; e < 4 && n + e < a.N; e++) v[e] += a.ws[s * plane + o + e];
    }
    for (int e = 0; e < 4 && n + e < a.N; e++) store_out<OT>(a, m, n + e, v[e]);
}

// The same reduction for N % 8 == 0 with 8 outputs per thread: 16-byte
// partial loads, vector scale / bias / residual loads and one 16-byte (fp16)
// or two 16-byte (fp32) stores.  The call moves a few MB at most and is
// bound by latency, or, with many splits over few outputs, by the few CUs
// its blocks occupy.  So the epilogue operands are requested first, the
// partials of up to G splits (2 G loads) go out together, and with GR > 1
// a block's threads form GR groups over the same 256 / GR chunks of 8
// outputs, group g summing the contiguous splits [S g / GR, S (g + 1) / GR)
// in order; the group sums are added in group order through LDS.  The
// result is ((sum of group 0) + sum of group 1) + ..., the same on every
// run for a given split count.
template <typename OT, int GR>
__global__ __launch_bounds__(256) void k_splitk_reduce8(LinArgs a)
{
    constexpr int G = 8;
    constexpr int CPB = 256 / GR;  // chunks per block, a multiple of 64: groups are whole waves
    __shared__ f4 part[GR > 1 ? GR - 1 : 1][CPB][2];
    const int t = threadIdx.x;
    const int g = t / CPB, lc = t % CPB;
    const int64_t q = (int64_t)blockIdx.x * CPB + lc;
    const int64_t per_row = a.N / 8;
    const bool live = q < a.M * per_row;
    const int64_t m = live ? q / per_row : 0, n = live ? (q - m * per_row) * 8 : 0;
    const int64_t o = m * a.N + n, plane = a.M * a.N;
    const int32_t s_lo = (int32_t)((int64_t)a.nsplit * g / GR), s_hi = (int32_t)((int64_t)a.nsplit * (g + 1) / GR);
    f4 s0 = {}, s1 = {}, b0 = {}, b1 = {};
    u4 r0 = {}, r1 = {};  // residual: 8 fp16 in r0, or 8 fp32 in r0 and r1
    if (g == 0 && live) {
        s0 = *reinterpret_cast<const f4*>(a.scales + n);
        s1 = *reinterpret_cast<const f4*>(a.scales + n + 4);
        if (a.bias) {
            b0 = *reinterpret_cast<const f4*>(a.bias + n);
            b1 = *reinterpret_cast<const f4*>(a.bias + n + 4);
        }
        if (a.res) {
            r0 = *reinterpret_cast<const u4*>(static_cast<const OT*>(a.res) + o);
            if constexpr (sizeof(OT) == 4) r1 = *reinterpret_cast<const u4*>(static_cast<const OT*>(a.res) + o + 4);
        }
    }
    f4 v0 = {}, v1 = {};
    if (live) {
        for (int32_t s = s_lo; s < s_hi; s += G) {
            f4 p[2 * G];
#pragma unroll
            for (int j = 0; j < G; j++)
                if (s + j < s_hi) {  // uniform over the wave
                    p[2 * j] = *reinterpret_cast<const f4*>(a.ws + (s + j) * plane + o);
                    p[2 * j + 1] = *reinterpret_cast<const f4*>(a.ws + (s + j) * plane + o + 4);
                }
#pragma unroll
            for (int j = 0; j < G; j++)
                if (s + j < s_hi) {
                    v0 += p[2 * j];
                    v1 += p[2 * j + 1];
                }
        }
    }
    if constexpr (GR > 1) {
        if (g > 0) {
            part[g - 1][lc][0] = v0;
            part[g - 1][lc][1] = v1;
        }
        __syncthreads();
        if (g > 0) return;
#pragma unroll
        for (int j = 0; j < GR - 1; j++) {
            v0 += part[j][lc][0];
            v1 += part[j][lc][1];
        }
    }
    if (!live) return;
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        v[e] = v0[e] * s0[e];
        v[4 + e] = v1[e] * s1[e];
    }
    if (a.bias) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] += b0[e];
            v[4 + e] += b1[e];
        }
    }
    if constexpr (sizeof(OT) == 2) {
        if (a.res) {
            const h8 r8 = __builtin_bit_cast(h8, r0);
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] += (float)r8[e];
        }
        h8 o8;
#pragma unroll
        for (int e = 0; e < 8; e++) o8[e] = (f16)v[e];
        *reinterpret_cast<h8*>(static_cast<f16*>(a.out) + o) = o8;
    } else {
        if (a.res) {
            const f4 x0 = __builtin_bit_cast(f4, r0), x1 = __builtin_bit_cast(f4, r1);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[e] += x0[e];
                v[4 + e] += x1[e];
            }
        }
        *reinterpret_cast<f4*>(static_cast<float*>(a.out) + o) = f4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f4*>(static_cast<float*>(a.out) + o + 4) = f4{v[4], v[5], v[6], v[7]};
    }
}

// Split groups per block of k_splitk_reduce8: more when few blocks of one
// group would carry many splits each.
int splitk_reduce_groups(int64_t M, int64_t N, int32_t nsplit)
{
    const int64_t blocks1 = (M * (N / 8) + 255) / 256;
    if (blocks1 >= 128) return 1;
    if (nsplit >= 8) return 4;
    return nsplit >= 4 ? 2 : 1;
}

template <typename OT>
static void reduce8_go(const LinArgs& a, hipStream_t s)
{
    const int gr = splitk_reduce_groups(a.M, a.N, a.nsplit);
    const int64_t chunks = a.M * (a.N / 8), cpb = 256 / gr;
    const dim3 grid((unsigned)((chunks + cpb - 1) / cpb));
    if (gr == 4) hipLaunchKernelGGL((k_splitk_reduce8<OT, 4>), grid, dim3(256), 0, s, a);
    else if (gr == 2) hipLaunchKernelGGL((k_splitk_reduce8<OT, 2>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_splitk_reduce8<OT, 1>), grid, dim3(256), 0, s, a);
}

int launch_splitk_reduce(const LinArgs& a, int out, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool vec = a.N % 8 == 0 && reinterpret_cast<uintptr_t>(a.out) % 16 == 0 &&
                     (!a.res || reinterpret_cast<uintptr_t>(a.res) % 16 == 0) &&
                     reinterpret_cast<uintptr_t>(a.scales) % 16 == 0 &&
                     (!a.bias || reinterpret_cast<uintptr_t>(a.bias) % 16 == 0);
    if (vec) {
        if (out == VVH_F32) reduce8_go<float>(a, s);
        else reduce8_go<f16>(a, s);
        return (int)hipGetLastError();
    }
    const int64_t threads = a.M * ((a.N + 3) / 4);
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (out == VVH_F32) hipLaunchKernelGGL((k_splitk_reduce<float>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_splitk_reduce<f16>), grid, dim3(256), 0, s, a);
    return (int)hipGetLastError();
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

template <int G>
static void skinny_launch(const LinArgs& a, int out, dim3 grid, hipStream_t s)
{
    if (out == VVH_F32) hipLaunchKernelGGL((k_skinny<float, G>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((k_skinny<f16, G>), grid, dim3(256), 0, s, a);
}

int launch_skinny(const LinArgs& a, int out, void* stream)
{
    const dim3 grid((unsigned)decode_blocks(a));
    if (a.M <= 16) skinny_launch<1>(a, out, grid, S(stream));
    else if (a.M <= 32) skinny_launch<2>(a, out, grid, S(stream));
    else skinny_launch<4>(a, out, grid, S(stream));
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

template <int MT, int XS, bool EARLY, int DEPTH, int FS, int NW = 4>
static void dot_launch(const LinArgs& a, int out, dim3 grid, size_t lds, hipStream_t s)
{
    // dot_fits(N, K) holds (checked by the runtime); M <= kDotMaxM, ksplit
    // <= 8, xparts <= kAttnMaxParts and xhd <= kAttnMergeMaxK (checked by
    // vvh_linear_q8_dev_attn) fit their fields
    const int32_t N = (int32_t)a.N, K = (int32_t)a.K;
    const int32_t mk = (int32_t)a.M | a.ksplit << 8;
    const int32_t xi = FS == kFirstAttn ? (a.xparts | a.xhd << 8) : 0;
    if (out == VVH_F32)
        hipLaunchKernelGGL((k_dot<float, MT, XS, EARLY, DEPTH, FS, NW>), grid, dim3(64 * NW), lds, s, a.w, a.inp,
                           a.scales, a.bias, a.res, N, K, mk, xi, a);
    else
        hipLaunchKernelGGL((k_dot<f16, MT, XS, EARLY, DEPTH, FS, NW>), grid, dim3(64 * NW), lds, s, a.w, a.inp,
                           a.scales, a.bias, a.res, N, K, mk, xi, a);
}

template <int MT, int XS, bool EARLY, int FS, int NW = 4>
static void dot_launch_d(const LinArgs& a, int out, int depth, dim3 grid, size_t lds, hipStream_t s)
{
    if (depth <= 2) dot_launch<MT, XS, EARLY, 2, FS, NW>(a, out, grid, lds, s);
    else if (depth <= 4) dot_launch<MT, XS, EARLY, 4, FS, NW>(a, out, grid, lds, s);
    else dot_launch<MT, XS, EARLY, 7, FS, NW>(a, out, grid, lds, s);
}

// first stages exist for early launches with staged activations only
template <int MT, int XS>
static void dot_launch_e(const LinArgs& a, int out, bool early, int fs, int depth, dim3 grid, size_t lds,
                         hipStream_t s)
{
    if (!early) {
        dot_launch_d<MT, XS, false, kFirstNone>(a, out, depth, grid, lds, s);
        return;
    }
    if constexpr (XS == kXLds) {
        if constexpr (MT <= 4) {
            if (fs == kFirstRms) return dot_launch_d<MT, true, true, kFirstRms>(a, out, depth, grid, lds, s);
            if (fs == kFirstRms4) return dot_launch_d<MT, true, true, kFirstRms4>(a, out, depth, grid, lds, s);
        }
        if constexpr (MT == 1)
            if (fs == kFirstAttn) return dot_launch_d<MT, true, true, kFirstAttn>(a, out, depth, grid, lds, s);
        if constexpr (MT <= 4) {  // dot_first_x: 1-4 rows
            if (fs == kFirstX1) return dot_launch_d<MT, true, true, kFirstX1>(a, out, depth, grid, lds, s);
            if (fs == kFirstX3) return dot_launch_d<MT, true, true, kFirstX3>(a, out, depth, grid, lds, s);
            if (fs == kFirstX5) return dot_launch_d<MT, true, true, kFirstX5>(a, out, depth, grid, lds, s);
        }
    }
    dot_launch_d<MT, XS, true, kFirstNone>(a, out, depth, grid, lds, s);
}

int launch_dot(const LinArgs& a, int out, bool early, int depth, void* stream)
{
    const dim3 grid((unsigned)dot_blocks(a));
    // early launches without an input stage stage one to four rows of
    // activations with a first stage (dot_first_x); more rows they load with the
    // weights (see dot_early).  The attention merge stage exists only as a
    // first stage (any block count).
    if (a.xop == 3) early = true;
    // (the activation tile, where it applies, takes precedence)
    const int64_t reread = dot_x_reread_bytes(a.M, a.N, a.K), wsteps = dot_wave_steps(a.K, a.ksplit);
    const bool tile = a.xop == 0 && dot_takes_x_tile(a.M, early, false, reread, wsteps);
    const int fx = a.xop == 0 && !tile ? dot_first_x(a.M, a.K, dot_blocks(a)) : kFirstNone;
    const bool xl = dot_x_in_lds(a.M, a.K) && (a.xop != 0 || !early || fx != kFirstNone);
    const int fs = !(early && xl) ? kFirstNone
                   : a.xop == 3 ? kFirstAttn
                   : a.xop == 1 ? dot_first_rms(a.M, a.K)
                   : fx;
    // the activation tile: MFMA path (M > 2), early launches loading the
    // activations with the weights, tiles re-reading many activation bytes
    const bool xt = dot_takes_x_tile(a.M, early, xl, reread, wsteps);
    hipStream_t st = S(stream);
    if (a.ksplit == 8) {
        // blocks of 8 waves (dot_split8): the plain MFMA path of an early
        // launch loading its activations with the weights, nothing else
        if (a.M <= 8 || a.M > kDotMaxM || !early || a.xop != 0 || xl || fs != kFirstNone)
            return (int)hipErrorInvalidValue;
        const size_t lds8 = 2 * (kDotRedBytes + kDotWtBytes + (xt ? kDotXtBytes : 0));
        if (xt) dot_launch_d<16, kXTile, true, kFirstNone, 8>(a, out, depth, grid, lds8, st);
        else dot_launch_d<16, kXDirect, true, kFirstNone, 8>(a, out, depth, grid, lds8, st);
        return (int)hipGetLastError();
    }
    const size_t lds = (xl ? dot_lds_bytes(a.M, a.K) : (size_t)kDotRedBytes) + (a.M > 2 ? kDotWtBytes : 0) +
                       (xt ? kDotXtBytes : 0);
    if (a.M <= 1) {
        if (xl) dot_launch_e<1, kXLds>(a, out, early, fs, depth, grid, lds, st);
        else dot_launch_e<1, kXDirect>(a, out, early, fs, depth, grid, lds, st);
    } else if (a.M <= 2) {
        if (xl) dot_launch_e<2, kXLds>(a, out, early, fs, depth, grid, lds, st);
        else dot_launch_e<2, kXDirect>(a, out, early, fs, depth, grid, lds, st);
    } else if (a.M <= 4) {
        if (xl) dot_launch_e<4, kXLds>(a, out, early, fs, depth, grid, lds, st);
        else if (xt) dot_launch_d<4, kXTile, true, kFirstNone>(a, out, depth, grid, lds, st);
        else dot_launch_e<4, kXDirect>(a, out, early, fs, depth, grid, lds, st);
    } else if (a.M <= 8) {
        if (xl) dot_launch_e<8, kXLds>(a, out, early, fs, depth, grid, lds, st);
        else if (xt) dot_launch_d<8, kXTile, true, kFirstNone>(a, out, depth, grid, lds, st);
        else dot_launch_e<8, kXDirect>(a, out, early, fs, depth, grid, lds, st);
    } else {
        if (xl) dot_launch_e<16, kXLds>(a, out, early, fs, depth, grid, lds, st);
        else if (xt) dot_launch_d<16, kXTile, true, kFirstNone>(a, out, depth, grid, lds, st);
        else dot_launch_e<16, kXDirect>(a, out, early, fs, depth, grid, lds, st);
    }
    return (int)hipGetLastError();
}

// The kernel arguments of a grouped launch besides the launch shape.
struct DotGroupArgs {
    int32_t b[3];
    int32_t count;
    int64_t pos;
    const LinArgs* table;
    const int32_t* block_prob;
    DotGroup g;
};

template <int MT, int XS, bool EARLY, int DEPTH, int FS, int EP>
static void dot_grouped_launch(const DotGroupArgs& k, int out, dim3 grid, size_t lds, hipStream_t s)
{
    if (out == VVH_F32)
        hipLaunchKernelGGL((k_dot_grouped<float, MT, XS, EARLY, DEPTH, FS, EP>), grid, dim3(256), lds, s, k.b[0],
                           k.b[1], k.b[2], k.count, k.pos, k.table, k.block_prob, k.g);
    else
        hipLaunchKernelGGL((k_dot_grouped<f16, MT, XS, EARLY, DEPTH, FS, EP>), grid, dim3(256), lds, s, k.b[0],
                           k.b[1], k.b[2], k.count, k.pos, k.table, k.block_prob, k.g);
}

template <int MT, int XS, bool EARLY, int FS, int EP = kEpiAny>
static void dot_grouped_launch_d(const DotGroupArgs& k, int out, int depth, dim3 grid, size_t lds, hipStream_t s)
{
    if (depth <= 2) dot_grouped_launch<MT, XS, EARLY, 2, FS, EP>(k, out, grid, lds, s);
    else if (depth <= 4) dot_grouped_launch<MT, XS, EARLY, 4, FS, EP>(k, out, grid, lds, s);
    else dot_grouped_launch<MT, XS, EARLY, 7, FS, EP>(k, out, grid, lds, s);
}

// plans take the RMSNorm first stage only (no attention merge stage); the
// epilogue kinds are compiled in one at a time for the decode step's
// single-row plans (q/k/v with RoPE, gate/up with SiLU-gating, the unfused
// q/k/v plan), every epilogue behind run-time tests otherwise
template <int MT, int FS>
static void dot_grouped_launch_rms(const DotGroupArgs& k, int out, int ep, int depth, dim3 grid, size_t lds,
                                   hipStream_t s)
{
    if constexpr (MT == 1) {
        if (ep == kEpiGlu) return dot_grouped_launch_d<MT, true, true, FS, kEpiGlu>(k, out, depth, grid, lds, s);
        if (ep == kEpiRope) return dot_grouped_launch_d<MT, true, true, FS, kEpiRope>(k, out, depth, grid, lds, s);
    }
    dot_grouped_launch_d<MT, true, true, FS>(k, out, depth, grid, lds, s);
}

template <int MT, int XS>
static void dot_grouped_launch_e(const DotGroupArgs& k, int out, bool early, int fs, int ep, int depth, dim3 grid,
                                 size_t lds, hipStream_t s)
{
    if (!early) {
        dot_grouped_launch_d<MT, XS, false, kFirstNone>(k, out, depth, grid, lds, s);
        return;
    }
    if constexpr (XS == kXLds && MT <= 4) {
        if (fs == kFirstRms) return dot_grouped_launch_rms<MT, kFirstRms>(k, out, ep, depth, grid, lds, s);
        if (fs == kFirstRms4) return dot_grouped_launch_rms<MT, kFirstRms4>(k, out, ep, depth, grid, lds, s);
    }
    if constexpr (MT == 1 && XS == kXDirect)
        if (ep == kEpiPlain) return dot_grouped_launch_d<MT, false, true, kFirstNone, kEpiPlain>(k, out, depth, grid, lds, s);
    dot_grouped_launch_d<MT, XS, true, kFirstNone>(k, out, depth, grid, lds, s);
}

int launch_dot_grouped(const LinArgs* dev_table, const int32_t* dev_block_prob, const LinArgs* args, int count,
                       int64_t total_blocks, int max_m, bool x_in_lds, size_t lds_bytes, int out, bool early,
                       int depth, int64_t pos, void* stream)
{
    const dim3 grid((unsigned)total_blocks);
    hipStream_t s = S(stream);
    // the MFMA path's code tiles, and its activation tiles where the
    // launch's tiles re-read many activation bytes (as launch_dot)
    int64_t reread = 0, wsteps = 0;
    for (int i = 0; i < count; ++i) {
        reread += dot_x_reread_bytes(args[i].M, args[i].N, args[i].K);
        wsteps = std::max(wsteps, dot_wave_steps(args[i].K, args[i].ksplit));
    }
    const bool xt = dot_takes_x_tile(max_m, early, x_in_lds, reread, wsteps);
    if (max_m > 2) lds_bytes += kDotWtBytes;
    if (xt) lds_bytes += kDotXtBytes;
    DotGroupArgs k{};
    k.count = count;
    k.pos = pos;
    k.table = dev_table;
    k.block_prob = dev_block_prob;
    for (int i = 0; i < 3; ++i) k.b[i] = INT32_MAX;
    if (count <= kDotInline)
        for (int i = 0; i < count; ++i) {
            k.g.p[i] = args[i];
            if (i > 0) k.b[i - 1] = args[i].block_begin;
        }
    // the RMSNorm first stage when every problem takes it (the larger of
    // the problems' forms; each problem's rows fit it)
    int fs = early && x_in_lds && count > 0 ? kFirstRms : kFirstNone;
    for (int i = 0; i < count && fs != kFirstNone; ++i) {
        const int f = args[i].xop == 1 ? dot_first_rms(args[i].M, args[i].K) : kFirstNone;
        fs = f == kFirstNone ? kFirstNone : std::max(fs, f);
    }
    // the one epilogue kind every problem takes, where there is one
    bool any_glu = false, all_glu = count > 0, any_rope = false;
    for (int i = 0; i < count; ++i) {
        any_glu = any_glu || args[i].glu != 0;
        all_glu = all_glu && args[i].glu != 0;
        any_rope = any_rope || args[i].rope != 0;
    }
    const int ep = all_glu && !any_rope ? kEpiGlu : !any_glu && any_rope ? kEpiRope : !any_glu ? kEpiPlain : kEpiAny;
    if (max_m <= 1) {
        if (x_in_lds) dot_grouped_launch_e<1, kXLds>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
        else dot_grouped_launch_e<1, kXDirect>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
    } else if (max_m <= 2) {
        if (x_in_lds) dot_grouped_launch_e<2, kXLds>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
        else dot_grouped_launch_e<2, kXDirect>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
    } else if (max_m <= 4) {
        if (x_in_lds) dot_grouped_launch_e<4, kXLds>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
        else if (xt) dot_grouped_launch_d<4, kXTile, true, kFirstNone>(k, out, depth, grid, lds_bytes, s);
        else dot_grouped_launch_e<4, kXDirect>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
    } else if (max_m <= 8) {
        if (x_in_lds) dot_grouped_launch_e<8, kXLds>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
        else if (xt) dot_grouped_launch_d<8, kXTile, true, kFirstNone>(k, out, depth, grid, lds_bytes, s);
        else dot_grouped_launch_e<8, kXDirect>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
    } else {
        if (x_in_lds) dot_grouped_launch_e<16, kXLds>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
        else if (xt) dot_grouped_launch_d<16, kXTile, true, kFirstNone>(k, out, depth, grid, lds_bytes, s);
        else dot_grouped_launch_e<16, kXDirect>(k, out, early, fs, ep, depth, grid, lds_bytes, s);
    }
    return (int)hipGetLastError();
}



template <typename OT, int D, int MR>
static void stream_launch(const StreamArgs& s, dim3 grid, hipStream_t st)
{
    if (s.mode == kStreamRange) hipLaunchKernelGGL((k_stream<OT, D, true, MR>), grid, dim3(256), 0, st, s);
    else hipLaunchKernelGGL((k_stream<OT, D, false, MR>), grid, dim3(256), 0, st, s);
}

template <int D, int MR>
static void stream_launch_out(const StreamArgs& s, int out, dim3 grid, hipStream_t st)
{
    if (out == VVH_F32) stream_launch<float, D, MR>(s, grid, st);
    else stream_launch<f16, D, MR>(s, grid, st);
}

int launch_stream(const StreamArgs& s, int depth, int max_m, int out, int64_t blocks, void* stream)
{
    const dim3 grid((unsigned)blocks);
    if (max_m <= 1) {
        if (depth >= 12) stream_launch_out<12, 1>(s, out, grid, S(stream));
        else stream_launch_out<8, 1>(s, out, grid, S(stream));
    } else {
        if (depth >= 12) stream_launch_out<12, 4>(s, out, grid, S(stream));
        else stream_launch_out<8, 4>(s, out, grid, S(stream));
    }
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
