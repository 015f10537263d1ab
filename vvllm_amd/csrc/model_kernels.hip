// Device kernels of the Backend operators around the int8 linears: the ops
// transformer_forward (include/vvllm/model/transformer.h:126-189) runs per
// decode step besides linear_q8.  Semantics follow BackendCPU
// (src/backend/backend_naive.cc) operation by operation, with activations in
// fp32 or fp16 (T) and every computation in fp32, one rounding on store.
//
//   k_eltwise    add / mul / silu / silu_mul            (:44-66, :293-300)
//   k_rms_norm   rows of RMSNorm, x / rms * w           (:68-76)
//   k_softmax    rows of softmax                        (:78-91)
//   k_rope       split-half rotary embedding, in place  (:93-137)
//   k_embedding  one table row, fp32 table             (:338-342)
//   k_attention  causal attention, one block per (head, query)  (:344-378)
//   k_dense      out = x @ W^T + bias (+ res), fp32 or fp16 W    (:139-156, :302-320)
//   k_matmul     out = A @ B, B [K, N]                  (:25-42)
//   k_sample     greedy sampling, first index of the max (src/sampler/sampler.cc:21-25),
//                and Gumbel-max temperature sampling (src/backend/cuda_kernels.cu:1228-1349)
//
// All are bandwidth- or latency-bound: per decode step they move kilobytes,
// except the dense LM head (the tied embedding, vocab x hidden weights) and
// attention over long contexts.
#include <hip/hip_runtime.h>

#include "common.h"
#include "device.h"

namespace vvh {

namespace {

template <typename T>
__device__ __forceinline__ float ldf(const T* p, int64_t i) { return (float)p[i]; }
template <typename T>
__device__ __forceinline__ void stf(T* p, int64_t i, float v) { p[i] = (T)v; }

__device__ __forceinline__ float silu_ref(float v) { return v * (1.0f / (1.0f + expf(-v))); }

// Block-wide sum / max over 256 threads (4 waves); `red` holds 4 floats.
__device__ __forceinline__ float block_sum(float v, float* red) { return block_sum256(v, red); }
__device__ __forceinline__ float block_max(float v, float* red)
{
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

}  // namespace

// ---------------------------------------------------------------------------
// elementwise
// ---------------------------------------------------------------------------
template <typename T, int OP>
__global__ __launch_bounds__(256) void k_eltwise(T* __restrict__ out, const T* __restrict__ x, const T* __restrict__ y,
                                                 int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float a = ldf(x, i);
        float r;
        if constexpr (OP == VVH_OP_ADD) r = a + ldf(y, i);
        else if constexpr (OP == VVH_OP_MUL) r = a * ldf(y, i);
        else if constexpr (OP == VVH_OP_SILU) r = silu_ref(a);
        else r = silu_mul_ref(a, ldf(y, i));  // silu_mul, backend_naive.cc:297-298
        stf(out, i, r);
    }
}

int launch_eltwise(int op, void* out, const void* x, const void* y, int64_t n, int dtype, void* stream)
{
    const int64_t want = (n + 255) / 256;
    const dim3 grid((unsigned)(want < 8192 ? (want > 0 ? want : 1) : 8192));
    hipStream_t s = static_cast<hipStream_t>(stream);
#define VVH_EW(T)                                                                                              \
    switch (op) {                                                                                              \
        case VVH_OP_ADD: hipLaunchKernelGGL((k_eltwise<T, VVH_OP_ADD>), grid, dim3(256), 0, s, (T*)out, (const T*)x, (const T*)y, n); break; \
        case VVH_OP_MUL: hipLaunchKernelGGL((k_eltwise<T, VVH_OP_MUL>), grid, dim3(256), 0, s, (T*)out, (const T*)x, (const T*)y, n); break; \
        case VVH_OP_SILU: hipLaunchKernelGGL((k_eltwise<T, VVH_OP_SILU>), grid, dim3(256), 0, s, (T*)out, (const T*)x, (const T*)y, n); break; \
        default: hipLaunchKernelGGL((k_eltwise<T, VVH_OP_SILU_MUL>), grid, dim3(256), 0, s, (T*)out, (const T*)x, (const T*)y, n); break; \
    }
    if (dtype == VVH_F16) { VVH_EW(f16) } else { VVH_EW(float) }
#undef VVH_EW
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm over `rows` rows of n: rms = sqrt(sum(x^2) / n + eps),
// out = x / rms * w (a division, as the reference; backend_naive.cc:68-76).
// One block of 4 waves per row; every wave sums the squares of the whole row
// in the order of rms_sumsq8 / wave_sum_xor (k_dot's RMSNorm input stages
// repeat it), so no barrier; thread (w, l) then writes chunk l + 64 w of 8
// values (and l + 64 w + 256 j for rows past 2048).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void rms_ld8(const T* p, float (&v)[8])
{
    if constexpr (sizeof(T) == 2) {
        const h8 h = *reinterpret_cast<const h8*>(p);
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (float)h[e];
    } else {
        const f4 a0 = *reinterpret_cast<const f4*>(p), a1 = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] = a0[e];
            v[4 + e] = a1[e];
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_rms_norm(T* __restrict__ out, const T* __restrict__ x,
                                                  const float* __restrict__ w, int64_t n, float eps)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const T* xr = x + (int64_t)blockIdx.x * n;
    T* orow = out + (int64_t)blockIdx.x * n;
    if (n <= 0) return;
    constexpr int RJ = 4;  // chunks of 8 per lane kept in registers: rows of up to 2048
    const bool vec = n % 8 == 0 && ((reinterpret_cast<uintptr_t>(xr) | reinterpret_cast<uintptr_t>(w) |
                                     reinterpret_cast<uintptr_t>(orow)) & 15) == 0;
    if (vec && n <= 64 * 8 * RJ) {
        // the lane's chunks requested at once (clamped into the row; past it
        // they add an exact 0), and the weights of the thread's own chunk
        const int64_t nc = n / 8, co = lane + 64 * wave, cw = co < nc ? co : nc - 1;
        float v[RJ][8];
#pragma unroll
        for (int j = 0; j < RJ; j++) rms_ld8(xr + 8 * (lane + 64 * j < nc ? lane + 64 * j : nc - 1), v[j]);
        const f4 w0 = *reinterpret_cast<const f4*>(w + 8 * cw), w1 = *reinterpret_cast<const f4*>(w + 8 * cw + 4);
        float ss = 0.0f, own[8];
#pragma unroll
        for (int j = 0; j < RJ; j++) {
            float z[8];
            const bool ok = lane + 64 * j < nc;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                z[e] = ok ? v[j][e] : 0.0f;
                own[e] = j == wave ? v[j][e] : (j == 0 ? 0.0f : own[e]);
            }
            ss = rms_sumsq8(ss, z);
        }
        const float rms = rms_of(wave_sum_xor(ss), n, eps);
        if (co < nc) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                stf(orow, 8 * co + e, rms_apply(own[e], rms, w0[e]));
                stf(orow, 8 * co + 4 + e, rms_apply(own[4 + e], rms, w1[e]));
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int64_t c = lane; 8 * c < n; c += 64) {
        float z[8];
#pragma unroll
        for (int e = 0; e < 8; e++) z[e] = 8 * c + e < n ? ldf(xr, 8 * c + e) : 0.0f;
        ss = rms_sumsq8(ss, z);
    }
    const float rms = rms_of(wave_sum_xor(ss), n, eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) stf(orow, i, rms_apply(ldf(xr, i), rms, w[i]));
}

int launch_rms_norm(void* out, const void* x, const float* w, int64_t rows, int64_t n, float eps, int dtype,
                    void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16)
        hipLaunchKernelGGL(k_rms_norm<f16>, dim3((unsigned)rows), dim3(256), 0, s, (f16*)out, (const f16*)x, w, n, eps);
    else
        hipLaunchKernelGGL(k_rms_norm<float>, dim3((unsigned)rows), dim3(256), 0, s, (float*)out, (const float*)x, w, n,
                           eps);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// softmax over `rows` rows of n: exp(x - max) / sum (backend_naive.cc:78-91)
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_softmax(T* __restrict__ out, const T* __restrict__ x, int64_t n)
{
    __shared__ float red[4];
    const T* xr = x + (int64_t)blockIdx.x * n;
    T* orow = out + (int64_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (int64_t i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, ldf(xr, i));
    mx = block_max(mx, red);
    float sum = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += 256) sum += expf(ldf(xr, i) - mx);
    sum = block_sum(sum, red);
    for (int64_t i = threadIdx.x; i < n; i += 256) stf(orow, i, expf(ldf(xr, i) - mx) / sum);
}

int launch_softmax(void* out, const void* x, int64_t rows, int64_t n, int dtype, void* stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16)
        hipLaunchKernelGGL(k_softmax<f16>, dim3((unsigned)rows), dim3(256), 0, s, (f16*)out, (const f16*)x, n);
    else
        hipLaunchKernelGGL(k_softmax<float>, dim3((unsigned)rows), dim3(256), 0, s, (float*)out, (const float*)x, n);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// RoPE, split-half pairs (i, i + D/2), in place on q [S, H, D] and k [S, KVH, D]
// at positions pos .. pos + S - 1 (backend_naive.cc:93-137): freq =
// 1 / theta^(2i / D), angle = position * freq in fp32.  One thread per pair.
// The fp32 angle multiplies any error of theta^(2i/D) by the position (30000
// x 1 ulp is ~1e-3 rad), so the power, cosine and sine are evaluated in fp64
// and rounded to fp32: the correctly rounded values, which is what the host
// libm's powf / cosf / sinf return.  The exponent, reciprocal, angle and
// rotation stay in the reference's fp32 operation order.
// ---------------------------------------------------------------------------
//
// APPEND (vvh_rope_append): the threads of the k pairs also store the rotated
// pair in the key cache row pos + s and copy the matching pair of v into the
// value cache row, the KVCache::append that follows rope in transformer_forward
// (transformer.h:145-160), without separate copies.
template <typename T, bool APPEND>
__global__ __launch_bounds__(256) void k_rope(T* __restrict__ q, T* __restrict__ k, int64_t S, int64_t H, int64_t KVH,
                                              int64_t D, int64_t pos, float theta, const T* __restrict__ v,
                                              T* __restrict__ kc, T* __restrict__ vc)
{
    const int64_t half = D / 2;
    const int64_t nq = S * H * half, total = nq + S * KVH * half;
    for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < total; g += (int64_t)gridDim.x * 256) {
        T* base;
        int64_t s, i, hs;
        const bool is_q = g < nq;
        if (is_q) {
            i = g % half;
            hs = g / half;  // s * H + h
            s = hs / H;
            base = q + hs * D;
        } else {
            const int64_t g2 = g - nq;
            i = g2 % half;
            hs = g2 / half;  // s * KVH + kvh
            s = hs / KVH;
            base = k + hs * D;
        }
        float f0, f1;
        rope_rotate(ldf(base, i), ldf(base, i + half), pos + s, i, D, theta, f0, f1);
        const T r0 = (T)f0, r1 = (T)f1;
        base[i] = r0;
        base[i + half] = r1;
        if constexpr (APPEND) {
            if (!is_q) {
                // row pos + s of the caches: hs * D - s * KVH * D = kvh * D
                const int64_t dst = (pos * KVH + hs) * D;
                kc[dst + i] = r0;
                kc[dst + i + half] = r1;
                vc[dst + i] = v[hs * D + i];
                vc[dst + i + half] = v[hs * D + i + half];
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_rope_freq(float* __restrict__ out, int64_t D, float theta)
{
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < D / 2) out[i] = rope_freq(i, D, theta);
}

int launch_rope_freq(float* out, int64_t D, float theta, void* stream)
{
    const int64_t n = D / 2;
    hipLaunchKernelGGL(k_rope_freq, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       out, D, theta);
    return (int)hipGetLastError();
}

__global__ __launch_bounds__(256) void k_rope_table(float2* __restrict__ out, const float* __restrict__ freq,
                                                    int64_t n, int64_t half)
{
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n) return;
    const int64_t p = e / half, i = e - p * half;
    float c, sn;
    rope_cs_freq(p, freq[i], c, sn);
    out[e] = make_float2(c, sn);
}

int launch_rope_table(float* out, const float* freq, int64_t positions, int64_t D, void* stream)
{
    const int64_t n = positions * (D / 2);
    hipLaunchKernelGGL(k_rope_table, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<float2*>(out), freq, n, D / 2);
    return (int)hipGetLastError();
}

int launch_rope(void* q, void* k, int64_t S, int64_t H, int64_t KVH, int64_t D, int64_t pos, float theta, int dtype,
                void* stream)
{
    const int64_t total = S * (H + KVH) * (D / 2);
    const int64_t want = (total + 255) / 256;
    const dim3 grid((unsigned)(want < 4096 ? (want > 0 ? want : 1) : 4096));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16)
        hipLaunchKernelGGL((k_rope<f16, false>), grid, dim3(256), 0, s, (f16*)q, (f16*)k, S, H, KVH, D, pos, theta,
                           nullptr, nullptr, nullptr);
    else
        hipLaunchKernelGGL((k_rope<float, false>), grid, dim3(256), 0, s, (float*)q, (float*)k, S, H, KVH, D, pos,
                           theta, nullptr, nullptr, nullptr);
    return (int)hipGetLastError();
}

int launch_rope_append(void* q, void* k, const void* v, void* kc, void* vc, int64_t S, int64_t H, int64_t KVH,
                       int64_t D, int64_t pos, float theta, int dtype, void* stream)
{
    const int64_t total = S * (H + KVH) * (D / 2);
    const int64_t want = (total + 255) / 256;
    const dim3 grid((unsigned)(want < 4096 ? (want > 0 ? want : 1) : 4096));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16)
        hipLaunchKernelGGL((k_rope<f16, true>), grid, dim3(256), 0, s, (f16*)q, (f16*)k, S, H, KVH, D, pos, theta,
                           (const f16*)v, (f16*)kc, (f16*)vc);
    else
        hipLaunchKernelGGL((k_rope<float, true>), grid, dim3(256), 0, s, (float*)q, (float*)k, S, H, KVH, D, pos,
                           theta, (const float*)v, (float*)kc, (float*)vc);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// embedding: out[0 .. hidden) = table[token][0 .. hidden) (fp32 table)
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_embedding(T* __restrict__ out, const float* __restrict__ table, int64_t token,
                                                   int64_t hidden)
{
    const float* row = table + token * hidden;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < hidden; i += (int64_t)gridDim.x * 256)
        stf(out, i, row[i]);
}

int launch_embedding(void* out, const float* table, int64_t token, int64_t hidden, int dtype, void* stream)
{
    const dim3 grid((unsigned)((hidden + 255) / 256 < 1024 ? (hidden + 255) / 256 : 1024));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16) hipLaunchKernelGGL(k_embedding<f16>, grid, dim3(256), 0, s, (f16*)out, table, token, hidden);
    else hipLaunchKernelGGL(k_embedding<float>, grid, dim3(256), 0, s, (float*)out, table, token, hidden);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Causal attention (backend_naive.cc:344-378): query s of q [n_q, H, D]
// attends to keys/values 0 .. len0 + s - 1 of k, v [*, KVH, D]; head h reads
// kv head h / (H / KVH).  score = (q . k) * scale; p = softmax(score) (max,
// exp, sum, then p / sum); out[s][h*D + d] = sum_t p_t v_t[d], in t order per
// thread slice.  One block of 256 threads per (head, query): the scores live
// in dynamic LDS (len floats); the weighted sum runs with D lanes over
// 256 / D key slices, reduced through LDS.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_attention(T* __restrict__ out, const T* __restrict__ q,
                                                   const T* __restrict__ k, const T* __restrict__ v, int64_t len0,
                                                   int64_t H, int64_t KVH, int64_t D, float scale)
{
    extern __shared__ float att_smem[];
    __shared__ float red[4];
    __shared__ float qs[256];
    const int64_t h = blockIdx.x, s = blockIdx.y;
    const int64_t len = len0 + s;
    const int64_t kvh = h / (H / KVH);
    const int64_t kv_stride = KVH * D;
    float* sc = att_smem;  // [len] scores, then probabilities; then [256 / D][D] partial sums
    const T* qrow = q + (s * H + h) * D;
    for (int64_t d = threadIdx.x; d < D; d += 256) qs[d] = ldf(qrow, d);
    __syncthreads();
    float mx = -INFINITY;
    for (int64_t t = threadIdx.x; t < len; t += 256) {
        const T* kr = k + t * kv_stride + kvh * D;
        float dot = 0.0f;
        for (int64_t d = 0; d < D; d++) dot += qs[d] * ldf(kr, d);
        const float x = dot * scale;
        sc[t] = x;
        mx = fmaxf(mx, x);
    }
    mx = block_max(mx, red);
    float sum = 0.0f;
    for (int64_t t = threadIdx.x; t < len; t += 256) {
        const float e = expf(sc[t] - mx);
        sc[t] = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    for (int64_t t = threadIdx.x; t < len; t += 256) sc[t] = sc[t] / sum;
    __syncthreads();
    // weighted sum of V: lane d of slice j covers keys j, j + slices, ...
    const int64_t slices = 256 / D;
    const int64_t d = threadIdx.x % D, j = threadIdx.x / D;
    float acc = 0.0f;
    if (j < slices)
        for (int64_t t = j; t < len; t += slices) acc += sc[t] * ldf(v + t * kv_stride + kvh * D, d);
    __syncthreads();
    float* part = att_smem;  // reuse: [slices][D]
    if (j < slices) part[j * D + d] = acc;
    __syncthreads();
    if (threadIdx.x < D) {
        float o = 0.0f;
        for (int64_t jj = 0; jj < slices; jj++) o += part[jj * D + threadIdx.x];
        stf(out, s * H * D + h * D + threadIdx.x, o);
    }
}

// ---------------------------------------------------------------------------
// Decode attention (one query per head, n_q = 1).  At decode positions the
// work is small (a few hundred K/V rows per layer) and latency-bound, so it
// is spread over many short blocks.  Block (g, c) takes kv head g and the
// keys [c * per_block, (c + 1) * per_block) for all G = H / KVH query heads
// that read kv head g, so each K and V row is loaded once for G heads.
//
// A key row is split over L lanes of 8 consecutive dims (L = D / 8 rounded
// up to a power of two), so a 256-thread block covers C = 256 / L keys per
// sub-chunk with one 16-byte load of K and of V per lane (two for fp32).
// Per sub-chunk:
//   scores   lane-partial dots for the G heads, xor-reduced over the L lanes,
//            into LDS (scores [G][C]); the V rows go to LDS as fp32;
//   softmax  per head (min(C, 64) lanes per head, so a wave serves 64 / C
//            heads at once when C < 64): running max m,
//            p = exp(s - m), running sum l = l * exp(m_old - m) + sum p;
//   P.V      thread (h, d) pairs: acc = acc * exp(m_old - m) + sum_j p_j v_j[d].
// One block per kv head writes out = acc / l; otherwise the block writes
// (m, l, acc[0..D)) to ws and k_attention_combine rescales the blocks to
// their common max.  D a multiple of 8 up to 128, G <= 16, k and v rows
// 16-byte aligned.
// ---------------------------------------------------------------------------
constexpr int kAttnMaxD = 128;
constexpr int kAttnMaxG = 16;
constexpr int kAttnOutPerThread = kAttnMaxG * kAttnMaxD / 256;

__host__ __device__ inline int attn_lanes(int D)
{
    int L = 1;
    while (L * 8 < D) L <<= 1;
    return L;
}

// 8 consecutive elements at p (16-byte aligned) as fp32
__device__ __forceinline__ void load8(const f16* p, float f[8])
{
    const h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int e = 0; e < 8; e++) f[e] = (float)v[e];
}
__device__ __forceinline__ void load8(const float* p, float f[8])
{
    const f4 a = *reinterpret_cast<const f4*>(p), b = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        f[e] = a[e];
        f[4 + e] = b[e];
    }
}

// ONE: the block's span is a single sub-chunk (per_block <= C), so there is
// nothing to prefetch.
template <typename T, bool ONE>
__global__ __launch_bounds__(256) void k_attention_decode(T* __restrict__ out, const T* __restrict__ q,
                                                          const T* __restrict__ k, const T* __restrict__ v,
                                                          int64_t len, int32_t H, int32_t KVH, int32_t D, float scale,
                                                          int64_t per_block, float* __restrict__ ws)
{
    __shared__ __align__(16) float ps[kAttnMaxG * 256];  // [h][j]: scores, then probabilities (G * C <= 16 * 256)
    __shared__ __align__(16) float vs[256 * 8];  // [j][d]: the sub-chunk's V rows (C * D <= 256 * 8)
    __shared__ __align__(16) float qs[kAttnMaxG * kAttnMaxD];  // [h][d]: the G query rows
    __shared__ float m_s[kAttnMaxG], l_s[kAttnMaxG], corr_s[kAttnMaxG];
    const int g = blockIdx.x, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int G = H / KVH;
    const int L = attn_lanes(D), C = 256 / L;
    const int j = tid / L, d0 = (tid % L) * 8;
    const bool dims_on = d0 < D;
    const int CL = C < 64 ? C : 64, R = 64 / CL, hl = lane / CL, il = lane - hl * CL;
    const int64_t kb = (int64_t)blockIdx.y * per_block;
    const int64_t ke = kb + per_block < len ? kb + per_block : len;
    const int64_t kvs = (int64_t)KVH * D;
    const int GD = G * D;
    // this thread's K/V rows (key t0 + j, dims d0 .. d0 + 7) of a sub-chunk,
    // loaded unconditionally from a clamped row; keys past the span and dims
    // past D are zeroed where the values are used, so the loads in flight
    // never depend on the key and the waits stay static
    const int dc = dims_on ? d0 : D - 8;
    auto load_kv = [&](int64_t t0, float (&kf)[8], float (&vf)[8]) {
        const int64_t t = t0 + j < ke ? t0 + j : ke - 1;
        load8(k + t * kvs + (int64_t)g * D + dc, kf);
        load8(v + t * kvs + (int64_t)g * D + dc, vf);
    };
    // the first sub-chunk's rows are requested before q is staged, so the
    // two round trips overlap
    float kf[8], vf[8];
    load_kv(kb, kf, vf);

    for (int i = tid; i < GD; i += 256) qs[i] = ldf(q, (int64_t)g * GD + i);
    float acc[kAttnOutPerThread];
#pragma unroll
    for (int i = 0; i < kAttnOutPerThread; i++) acc[i] = 0.0f;
    if (tid < G) {
        m_s[tid] = -INFINITY;
        l_s[tid] = 0.0f;
    }
    __syncthreads();

    for (int64_t t0 = kb; t0 < ke; t0 += C) {
        const int64_t t = t0 + j;
        const bool key_on = t < ke;
        // the next sub-chunk's rows, one sub-chunk ahead
        float kn[8], vn[8];
        if constexpr (!ONE) load_kv(t0 + C, kn, vn);
        const bool on = key_on && dims_on;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kf[e] = on ? kf[e] : 0.0f;
            vf[e] = on ? vf[e] : 0.0f;
        }
        float sc[kAttnMaxG];
#pragma unroll
        for (int h = 0; h < kAttnMaxG; h++) {
            float a = 0.0f;
            if (h < G) {
                if (dims_on) {
                    const f4 q0 = *reinterpret_cast<const f4*>(qs + h * D + d0);
                    const f4 q1 = *reinterpret_cast<const f4*>(qs + h * D + d0 + 4);
#pragma unroll
                    for (int e = 0; e < 4; e++) a += q0[e] * kf[e] + q1[e] * kf[4 + e];
                }
                a = group_sum(a, L);
            }
            sc[h] = a;
        }
        __syncthreads();  // the previous sub-chunk's P.V has read ps and vs
        if (tid % L == 0) {
#pragma unroll
            for (int h = 0; h < kAttnMaxG; h++)
                if (h < G) ps[h * C + j] = key_on ? sc[h] * scale : -INFINITY;
        }
        if (dims_on) {
#pragma unroll
            for (int e = 0; e < 8; e++) vs[j * D + d0 + e] = vf[e];
        }
        __syncthreads();
        // R heads per wave at once, CL lanes per head
        for (int h0 = wv * R; h0 < G; h0 += 4 * R) {
            const int h = h0 + hl;
            const bool hon = h < G;
            float mc = -INFINITY;
            if (hon)
                for (int i = il; i < C; i += CL) mc = fmaxf(mc, ps[h * C + i]);
            mc = group_max(mc, CL);
            const float mo = hon ? m_s[h] : 0.0f, mn = fmaxf(mo, mc);  // mc is finite: the sub-chunk has a key
            float sum = 0.0f;
            if (hon)
                for (int i = il; i < C; i += CL) {
                    const float e = expf(ps[h * C + i] - mn);
                    ps[h * C + i] = e;
                    sum += e;
                }
            sum = group_sum(sum, CL);
            if (hon && il == 0) {
                const float cr = expf(mo - mn);  // 0 on the first sub-chunk
                corr_s[h] = cr;
                l_s[h] = l_s[h] * cr + sum;
                m_s[h] = mn;
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kAttnOutPerThread; i++) {
            const int o = tid + 256 * i;
            if (o < GD) {
                const int h = o / D, d = o - h * D;
                float a = acc[i] * corr_s[h];
                for (int jj = 0; jj < C; jj++) a += ps[h * C + jj] * vs[jj * D + d];
                acc[i] = a;
            }
        }
        if constexpr (!ONE) {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kf[e] = kn[e];
                vf[e] = vn[e];
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kAttnOutPerThread; i++) {
        const int o = tid + 256 * i;
        if (o < GD) {
            const int h = o / D, d = o - h * D, head = g * G + h;
            if (gridDim.y == 1) {
                stf(out, (int64_t)head * D + d, acc[i] / l_s[h]);
            } else {
                float* w = ws + ((int64_t)blockIdx.y * H + head) * (D + 2);
                w[2 + d] = acc[i];
                if (d == 0) {
                    w[0] = m_s[h];
                    w[1] = l_s[h];
                }
            }
        }
    }
}

// out[h][d] = sum_c e^(m_c - M) o_c[d] / sum_c e^(m_c - M) l_c, M = max_c m_c.
// Block per head, one pass over the partials: thread (s, d) merges the
// blocks c = s, s + S, ... (S = blockDim.x / D) into a running maximum and sums
// rescaled to it (the online-softmax merge); the S groups then merge the
// same way through LDS.
template <typename T>
__global__ __launch_bounds__(1024) void k_attention_combine(T* __restrict__ out, const float* __restrict__ ws,
                                                            int32_t blocks, int32_t H, int32_t D)
{
    __shared__ float sm[1024], sn[1024], sd[1024];
    const int h = blockIdx.x, tid = threadIdx.x;
    const int S = (int)blockDim.x / D, s = tid / D, d = tid - s * D;
    float M = -INFINITY, num = 0.0f, den = 0.0f;
    if (s < S) {
#pragma unroll 4
        for (int c = s; c < blocks; c += S) {
            const float* w = ws + ((int64_t)c * H + h) * (D + 2);
            const float m = w[0], l = w[1], o = w[2 + d];
            const float mn = fmaxf(M, m);          // m is finite: every block has a key
            const float a = expf(M - mn), b = expf(m - mn);  // a = 0 on the first block
            num = num * a + o * b;
            den = den * a + l * b;
            M = mn;
        }
    }
    sm[tid] = M;
    sn[tid] = num;
    sd[tid] = den;
    __syncthreads();
    if (tid < D) {
        float mt = -INFINITY;
        for (int g = 0; g < S; g++) mt = fmaxf(mt, sm[g * D + tid]);
        float a = 0.0f, b = 0.0f;
        for (int g = 0; g < S; g++) {
            const float f = expf(sm[g * D + tid] - mt);  // 0 for a group without blocks
            a += sn[g * D + tid] * f;
            b += sd[g * D + tid] * f;
        }
        stf(out, (int64_t)h * D + tid, a / b);
    }
}

// ---------------------------------------------------------------------------
// Decode attention on the matrix cores: fp16 q, K and V, head_dim 64 or 128,
// at most 16 query heads per kv head.  Same arithmetic as above (fp32 scores,
// softmax and sums) with no runtime-shaped loops: a span of one key and a
// span of 256 cost the same few dependent steps.
//
// Grid (KVH, nb), W = kDecWaves waves per block (4 or 8).  Block (g, b) takes kv head
// g and the keys [b * per_block, (b + 1) * per_block); its span is cut into
// chunks of 64 keys and wave w takes chunks w, w + W, ...  Per chunk, one
// wave:
//   S^T = K . q^T   v_mfma_f32_16x16x32_f16 per 16-key tile and 32 dims:
//                   A = K rows (lane: key l % 16, the 8 dims of group l / 16,
//                   one 16-byte load), B = the G query rows of the kv head
//                   padded with zero rows to 16 columns.  Per lane the result
//                   is head l % 16's scores for keys 4 (l / 16) + 0..3 of each
//                   tile;
//   softmax         online, per head: max and sum over the lane's 16 scores and
//                   the 4 lanes of the head (exp2 of scores pre-scaled by
//                   log2 e);
//   O^T += V^T P^T  A = V^T (16 dims x 32 keys), gathered from the chunk's V
//                   rows staged in the wave's LDS region; B = the lane's own
//                   probabilities: the 8 keys a lane supplies to a 32-key step
//                   are its scores of two tiles, so P needs no shuffles.  P is
//                   split into fp16 hi + lo (two products), keeping ~22 bits.
// The K-dimension order inside an MFMA is the same for A and B, so any
// assignment of dims (or keys) to a lane's 8 slots that A and B share gives
// the same sums.  The W waves merge their (max, sum, O) through LDS.  With one
// block per kv head the block writes the output; otherwise each block writes
// its partial (max, sum, O) to ws, and the last block of the kv head to arrive
// (a per-kv-head counter in cnt, left at zero again for the next call) merges
// the nb partials and writes the output: one launch either way.
// ---------------------------------------------------------------------------
constexpr int kDecChunk = 64;  // keys per wave and chunk

typedef _Float16 h4v __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950): an 8-byte LDS read per lane, transposed in
// groups of 16 lanes (lane i's element j is lane 4j + i/4's element i % 4).
// p must point into LDS, 8-byte aligned.
__device__ __forceinline__ h4v lds_read_tr16(const _Float16* p)
{
    typedef short s4v __attribute__((ext_vector_type(4)));
    const s4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4v*)(p));
    return __builtin_bit_cast(h4v, v);
}

// The G query rows of kv head g as B operands of the score MFMAs (lane:
// head l % 16, dims 32 s + 8 (l / 16) .. + 7; rows past G are zero).
template <int D>
__device__ __forceinline__ void attn_load_q(const f16* __restrict__ q, int g, int G, int lane, h8 (&qb)[D / 32])
{
    const int r = lane & 15, gr = lane >> 4;
#pragma unroll
    for (int s = 0; s < D / 32; s++) {
        h8 z = {};
        qb[s] = r < G ? *reinterpret_cast<const h8*>(q + ((int64_t)g * G + r) * D + 32 * s + 8 * gr) : z;
    }
}

// One wave's share of a kv head's span: the chunks of 64 keys starting at
// c0, c0 + cstep, ... below ke, folded into head (lane % 16)'s running max m
// (log2 units), sum l and O^T fragments o.  vw: the wave's LDS region of
// kDecChunk rows of D + 4 halves.  kh / vh: the kv head's column in the K / V
// caches (row stride kvs).
template <int D>
__device__ __forceinline__ void attn_wave_chunks(const f16* __restrict__ kh, const f16* __restrict__ vh, int64_t kvs,
                                                 const h8 (&qb)[D / 32], int64_t c0, int64_t cstep, int64_t ke,
                                                 float scale_log2, _Float16* vw, int lane, float& m, float& l,
                                                 f4 (&o)[D / 16])
{
    constexpr int DS = D / 32;              // 32-dim steps of a score tile
    constexpr int DE = D / 16;              // 16-dim tiles of O^T
    constexpr int VP = D + 4;               // V row pitch in LDS (halves): 2-byte gathers conflict-free
    constexpr int VR = kDecChunk * D / 512; // 16-byte pieces of a chunk's V rows per lane
    const int r = lane & 15, gr = lane >> 4;
    for (; c0 < ke; c0 += cstep) {
        // every row index clamped into the span: rows past it are loaded from
        // key ke - 1 and weighted 0.  Plain (cached) loads: a layer's K/V rows
        // are read again at the next token while the weights in between
        // stream past the caches non-temporally (Qwen2.5-0.5B decode step at
        // position 511: 719 -> 701 us per token against non-temporal loads)
        h8 ka[4][DS], vr[VR];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int64_t key = c0 + 16 * t + r < ke ? c0 + 16 * t + r : ke - 1;
#pragma unroll
            for (int s = 0; s < DS; s++)
                ka[t][s] = *reinterpret_cast<const h8*>(kh + key * kvs + 32 * s + 8 * gr);
        }
#pragma unroll
        for (int i = 0; i < VR; i++) {
            const int p = i * 64 + lane, row = p / (D / 8), col = (p % (D / 8)) * 8;
            const int64_t key = c0 + row < ke ? c0 + row : ke - 1;
            vr[i] = *reinterpret_cast<const h8*>(vh + key * kvs + col);
        }
        f4 sc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            sc[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < DS; s++) sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[t][s], qb[s], sc[t], 0, 0, 0);
        }
        float cm = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float x = c0 + 16 * t + 4 * gr + i < ke ? sc[t][i] * scale_log2 : -INFINITY;
                sc[t][i] = x;
                cm = fmaxf(cm, x);
            }
        cm = max_x16(cm);
        cm = max_x32(cm);  // finite: key c0 is in the span
        const float mn = fmaxf(m, cm), corr = exp2f(m - mn);  // corr = 0 on the first chunk
        float ps = 0.0f;
        h8 ph[2], pl[2];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float p = exp2f(sc[2 * u + j / 4][j % 4] - mn);
                ps += p;
                const _Float16 hi = (_Float16)p;
                ph[u][j] = hi;
                pl[u][j] = (_Float16)(p - (float)hi);
            }
        ps = sum_x16(ps);
        ps = sum_x32(ps);
        l = l * corr + ps;
        m = mn;
#pragma unroll
        for (int e = 0; e < DE; e++) o[e] *= corr;
        // the chunk's V rows into the wave's region; one wave's LDS accesses
        // complete in order, so the gathers below read these rows, and the
        // next chunk's writes follow this chunk's gathers
#pragma unroll
        for (int i = 0; i < VR; i++) {
            const int p = i * 64 + lane, row = p / (D / 8), col = (p % (D / 8)) * 8;
            *reinterpret_cast<h4v*>(vw + row * VP + col) = h4v{vr[i][0], vr[i][1], vr[i][2], vr[i][3]};
            *reinterpret_cast<h4v*>(vw + row * VP + col + 4) = h4v{vr[i][4], vr[i][5], vr[i][6], vr[i][7]};
        }
        // A operand of the PV MFMAs: lane (r, gr) holds V[key][16e + r] for
        // keys 32u + 4gr + j and 32u + 16 + 4gr + j, j < 4.  Two LDS transpose
        // reads give them: in each group of 16 lanes, lane i's element j
        // comes from lane 4j + i/4's 8-byte piece, element i % 4, so lane s
        // of the group points at 4 consecutive dims (16e + 4(s % 4)) of key
        // row 32u + 4gr + s / 4 (and of the row 16 keys on).
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int e = 0; e < DE; e++) {
                const _Float16* src = vw + (32 * u + 4 * gr + (r >> 2)) * VP + 16 * e + 4 * (r & 3);
                const h4v lo = lds_read_tr16(src), hi = lds_read_tr16(src + 16 * VP);
                const h8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph[u], o[e], 0, 0, 0);
                o[e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl[u], o[e], 0, 0, 0);
            }
    }
}

// What the first loads depend on comes first (q, k, v, the key range, the
// head layout: 14 dwords, preloaded into registers at dispatch); G = H / KVH.
template <int D, int kDecWaves>
__global__ __launch_bounds__(64 * kDecWaves) void k_attention_decode_mfma(const f16* __restrict__ q,
                                                               const f16* __restrict__ k, const f16* __restrict__ v,
                                                               int64_t len, int64_t per_block, int32_t KVH, int32_t G,
                                                               float scale_log2, f16* __restrict__ out,
                                                               float* __restrict__ ws, unsigned* __restrict__ cnt)
{
    constexpr int DE = D / 16;              // 16-dim tiles of O^T
    constexpr int VP = D + 4;               // V row pitch in LDS (halves)
    constexpr int OP = D + 4;               // O row pitch in LDS (floats)
    static_assert(kDecWaves * kDecChunk * VP * 2 >= kDecWaves * 16 * OP * 4, "O aliases the V regions");
    __shared__ __align__(16) _Float16 vs[kDecWaves * kDecChunk * VP];
    __shared__ float wm[kDecWaves][16], wl[kDecWaves][16];
    __shared__ int last_s;
    const int g = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63, r = lane & 15, gr = lane >> 4;
    const int H = G * KVH;
    const int64_t kvs = (int64_t)KVH * D;
    const int64_t kb = (int64_t)blockIdx.y * per_block;
    const int64_t ke = kb + per_block < len ? kb + per_block : len;

    h8 qb[D / 32];
    attn_load_q<D>(q, g, G, lane, qb);
    float m = -INFINITY, l = 0.0f;  // head r's running max (log2 units) and sum
    f4 o[DE];
#pragma unroll
    for (int e = 0; e < DE; e++) o[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    attn_wave_chunks<D>(k + (int64_t)g * D, v + (int64_t)g * D, kvs, qb, kb + (int64_t)w * kDecChunk,
                        (int64_t)kDecWaves * kDecChunk, ke, scale_log2, vs + w * kDecChunk * VP, lane, m, l, o);

    // merge the waves: (max, sum) per head, O^T per head as rows of os
    __syncthreads();  // every wave is done with its V region
    float* os = reinterpret_cast<float*>(vs);
    if (gr == 0) {
        wm[w][r] = m;
        wl[w][r] = l;
    }
#pragma unroll
    for (int e = 0; e < DE; e++) *reinterpret_cast<f4*>(os + (w * 16 + r) * OP + 16 * e + 4 * gr) = o[e];
    __syncthreads();
    const bool split = gridDim.y > 1;
    for (int idx = tid; idx < G * D; idx += 64 * kDecWaves) {
        const int h = idx / D, d = idx - h * D;
        float M = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kDecWaves; ww++) M = fmaxf(M, wm[ww][h]);  // finite: wave 0 has a key
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kDecWaves; ww++)  // a wave without keys adds exact zeros
            attn_merge_add(num, den, wm[ww][h], M, os[(ww * 16 + h) * OP + d], wl[ww][h]);
        if (!split) {
            out[((int64_t)g * G + h) * D + d] = (f16)(num / den);
        } else {
            float* pw = ws + ((int64_t)blockIdx.y * H + (int64_t)g * G + h) * (D + 2);
            pw[2 + d] = num;
            if (d == 0) {
                pw[0] = M;
                pw[1] = den;
            }
        }
    }
    if (!split) return;
    // the partials visible device-wide before the block counts itself in
    __threadfence();
    __syncthreads();
    if (tid == 0) last_s = atomicAdd(cnt + g, 1u) == gridDim.y - 1;
    __syncthreads();
    if (!last_s) return;
    __threadfence();  // the other blocks' partials, not stale cached lines
    const int nb = (int)gridDim.y;
    for (int idx = tid; idx < G * D; idx += 64 * kDecWaves) {
        const int h = idx / D, d = idx - h * D;
        const float* pw = ws + ((int64_t)g * G + h) * (D + 2);
        const int64_t step = (int64_t)H * (D + 2);
        float M = -INFINITY, num = 0.0f, den = 0.0f;
#pragma unroll 4
        for (int b = 0; b < nb; b++) {
            const float mb = pw[b * step], lb = pw[b * step + 1], ob = pw[b * step + 2 + d];
            const float mx = fmaxf(M, mb);  // mb is finite: every block has a key
            const float a = exp2f(M - mx), c = exp2f(mb - mx);
            num = num * a + ob * c;
            den = den * a + lb * c;
            M = mx;
        }
        out[((int64_t)g * G + h) * D + d] = (f16)(num / den);
    }
    if (tid == 0) cnt[g] = 0u;  // ready for the next call on this stream
}

// Decode attention as per-wave parts, for spans that k_attention_decode_mfma
// takes in one block of W waves (nb == 1): block (g, w) is one wave doing
// what wave w of that block does (the chunks w, w + W, ... of kv head g, the
// same wave body) and writes, for each query head h = g G + r of the kv
// head, its running max m, sum l and O (D values) to the part row
// parts + (w H + h) (D + 4) as [O, m, l, -, -].  Merging the W part rows of a
// head in part order (attn_merge_add, then num / den) repeats the block's
// merge of its waves, so the output has the bits of the one-launch kernel;
// the merge runs in the consumer (k_dot input stage 3).  One wave per block
// spreads a kv head's K/V rows over W CUs instead of one.
template <int D>
__global__ __launch_bounds__(64) void k_attention_parts(const f16* __restrict__ q, const f16* __restrict__ k,
                                                        const f16* __restrict__ v, int64_t len, int32_t KVH,
                                                        int32_t G, float scale_log2, float* __restrict__ parts)
{
    constexpr int DE = D / 16;
    __shared__ __align__(16) _Float16 vs[kDecChunk * (D + 4)];
    const int g = blockIdx.x, w = blockIdx.y, lane = threadIdx.x, r = lane & 15, gr = lane >> 4;
    const int W = (int)gridDim.y, H = G * KVH;
    h8 qb[D / 32];
    attn_load_q<D>(q, g, G, lane, qb);
    float m = -INFINITY, l = 0.0f;
    f4 o[DE];
#pragma unroll
    for (int e = 0; e < DE; e++) o[e] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    attn_wave_chunks<D>(k + (int64_t)g * D, v + (int64_t)g * D, (int64_t)KVH * D, qb, (int64_t)w * kDecChunk,
                        (int64_t)W * kDecChunk, len, scale_log2, vs, lane, m, l, o);
    if (r < G) {
        float* pr = parts + ((int64_t)w * H + (int64_t)g * G + r) * (D + 4);
#pragma unroll
        for (int e = 0; e < DE; e++) *reinterpret_cast<f4*>(pr + 16 * e + 4 * gr) = o[e];
        if (gr == 0) {
            pr[D] = m;
            pr[D + 1] = l;
        }
    }
}

__global__ void k_zero_u32(unsigned* __restrict__ p, int64_t n)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Two copies of n bytes in one launch (the K and V rows of a cache append):
// 16-byte chunks when every pointer and n allow it, else bytes.
template <typename U>
__global__ __launch_bounds__(256) void k_copy2(U* __restrict__ d0, const U* __restrict__ s0, U* __restrict__ d1,
                                              const U* __restrict__ s1, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < 2 * n; i += (int64_t)gridDim.x * 256) {
        if (i < n) d0[i] = s0[i];
        else d1[i - n] = s1[i - n];
    }
}

int launch_copy2(void* d0, const void* s0, void* d1, const void* s1, int64_t bytes, void* stream)
{
    if (bytes <= 0) return 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool v16 = bytes % 16 == 0 && ((reinterpret_cast<uintptr_t>(d0) | reinterpret_cast<uintptr_t>(s0) |
                                          reinterpret_cast<uintptr_t>(d1) | reinterpret_cast<uintptr_t>(s1)) & 15) == 0;
    const int64_t n = v16 ? bytes / 16 : bytes;
    const unsigned blocks = (unsigned)std::min<int64_t>((2 * n + 255) / 256, 1024);
    if (v16)
        hipLaunchKernelGGL(k_copy2<u4>, dim3(blocks), dim3(256), 0, s, (u4*)d0, (const u4*)s0, (u4*)d1, (const u4*)s1,
                           n);
    else
        hipLaunchKernelGGL(k_copy2<uint8_t>, dim3(blocks), dim3(256), 0, s, (uint8_t*)d0, (const uint8_t*)s0,
                           (uint8_t*)d1, (const uint8_t*)s1, n);
    return (int)hipGetLastError();
}

int launch_zero_u32(unsigned* p, int64_t n, void* stream)
{
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_zero_u32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       p, n);
    return (int)hipGetLastError();
}

bool attention_decode_ok(const void* k, const void* v, int64_t len, int64_t H, int64_t KVH, int64_t D)
{
    return D % 8 == 0 && D <= kAttnMaxD && H / KVH <= kAttnMaxG && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(v) % 16 == 0 && len <= attention_decode_max_len();
}

int64_t attention_decode_max_len() { return (int64_t)1 << 30; }

// Keys per block of the lane kernel: whole sub-chunks, as few as keep at
// most ~512 blocks in the grid (two per CU), so short spans get one
// sub-chunk per block.
static int64_t attn_per_block(int64_t len, int64_t KVH, int64_t D)
{
    const int64_t C = 256 / attn_lanes((int)D);
    const int64_t chunks = (len + C - 1) / C;
    const int64_t nb_max = std::max<int64_t>(1, 512 / KVH);
    const int64_t per = (chunks + nb_max - 1) / nb_max;
    return per * C;
}

// The matrix-core kernel takes spans of up to 8 chunks of 64 keys in one
// block per kv head, one chunk per wave (4 waves up to 4 chunks, else 8), with
// no cross-block merge.  Longer spans take 4-wave blocks, one chunk per wave
// while that keeps at most 64 blocks per kv head and ~256 blocks in all,
// several beyond.  (Graph-replayed, Qwen2.5-0.5B shapes: a wave's second
// chunk costs ~2 us, the cross-block merge ~3.4 us, so 8 waves in one block
// win at 512 keys and 4-wave blocks at 1024 and beyond.)
AttnDecodePlan attention_decode_plan(const void* q, int64_t len, int64_t H, int64_t KVH, int64_t D, int dtype)
{
    AttnDecodePlan p{};
    p.mfma = dtype == VVH_F16 && (D == 64 || D == 128) && H / KVH <= 16 && KVH <= kAttnCounters &&
             reinterpret_cast<uintptr_t>(q) % 16 == 0;
    if (p.mfma) {
        const int64_t chunks = (len + kDecChunk - 1) / kDecChunk;
        if (chunks <= 8) {
            p.waves = chunks <= 4 ? 4 : 8;
            p.per_block = p.waves * kDecChunk;
        } else {
            p.waves = 4;
            const int64_t nb_cap = std::min<int64_t>(64, std::max<int64_t>(1, 256 / KVH));
            const int64_t per_wave = (chunks + 4 * nb_cap - 1) / (4 * nb_cap);
            p.per_block = per_wave * 4 * kDecChunk;
        }
    } else {
        p.per_block = attn_per_block(len, KVH, D);
    }
    p.nb = (len + p.per_block - 1) / p.per_block;
    return p;
}

int launch_attention_parts(float* parts, const void* q, const void* k, const void* v, int64_t len, int64_t H,
                           int64_t KVH, int64_t D, float scale, int nparts, void* stream)
{
    const dim3 grid((unsigned)KVH, (unsigned)nparts);
    const float sl = (float)((double)scale * 1.4426950408889634);  // as launch_attention_decode
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (D == 64)
        hipLaunchKernelGGL(k_attention_parts<64>, grid, dim3(64), 0, s, (const f16*)q, (const f16*)k, (const f16*)v,
                           len, (int32_t)KVH, (int32_t)(H / KVH), sl, parts);
    else
        hipLaunchKernelGGL(k_attention_parts<128>, grid, dim3(64), 0, s, (const f16*)q, (const f16*)k, (const f16*)v,
                           len, (int32_t)KVH, (int32_t)(H / KVH), sl, parts);
    return (int)hipGetLastError();
}

int64_t attention_decode_ws_floats(const AttnDecodePlan& p, int64_t H, int64_t D)
{
    return p.nb > 1 ? p.nb * H * (D + 2) : 0;
}

// Combine block: D x S threads, S (a power of two, 1 <= S <= 1024 / D) the
// smallest that leaves each thread at most 4 partials, so long spans fold in
// parallel instead of in one long chain per thread.
static unsigned combine_threads(int64_t nb, int64_t D)
{
    int64_t S = 1;
    while (S * 4 < nb && S * 2 * D <= 1024) S *= 2;
    return (unsigned)(S * D);
}

int launch_attention_decode(const AttnDecodePlan& p, void* out, const void* q, const void* k, const void* v,
                            int64_t len, int64_t H, int64_t KVH, int64_t D, float scale, float* ws, unsigned* cnt,
                            int dtype, void* stream)
{
    const int64_t per = p.per_block, nb = p.nb;
    const dim3 grid((unsigned)KVH, (unsigned)nb);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (p.mfma) {
        const float sl = (float)((double)scale * 1.4426950408889634);  // scores in log2 units
        auto go = [&](auto kern) {
            hipLaunchKernelGGL(kern, grid, dim3(64 * p.waves), 0, s, (const f16*)q, (const f16*)k, (const f16*)v,
                               len, per, (int32_t)KVH, (int32_t)(H / KVH), sl, (f16*)out, ws, cnt);
        };
        if (D == 64)
            p.waves == 8 ? go(k_attention_decode_mfma<64, 8>) : go(k_attention_decode_mfma<64, 4>);
        else
            p.waves == 8 ? go(k_attention_decode_mfma<128, 8>) : go(k_attention_decode_mfma<128, 4>);
        return (int)hipGetLastError();
    }
    const bool one = per <= 256 / attn_lanes((int)D);  // one sub-chunk per block
    if (dtype == VVH_F16) {
        if (one)
            hipLaunchKernelGGL((k_attention_decode<f16, true>), grid, dim3(256), 0, s, (f16*)out, (const f16*)q,
                               (const f16*)k, (const f16*)v, len, (int32_t)H, (int32_t)KVH, (int32_t)D, scale, per, ws);
        else
            hipLaunchKernelGGL((k_attention_decode<f16, false>), grid, dim3(256), 0, s, (f16*)out, (const f16*)q,
                               (const f16*)k, (const f16*)v, len, (int32_t)H, (int32_t)KVH, (int32_t)D, scale, per, ws);
        if (nb > 1)
            hipLaunchKernelGGL(k_attention_combine<f16>, dim3((unsigned)H), dim3(combine_threads(nb, D)), 0, s, (f16*)out, ws,
                               (int32_t)nb, (int32_t)H, (int32_t)D);
    } else {
        if (one)
            hipLaunchKernelGGL((k_attention_decode<float, true>), grid, dim3(256), 0, s, (float*)out,
                               (const float*)q, (const float*)k, (const float*)v, len, (int32_t)H, (int32_t)KVH,
                               (int32_t)D, scale, per, ws);
        else
            hipLaunchKernelGGL((k_attention_decode<float, false>), grid, dim3(256), 0, s, (float*)out,
                               (const float*)q, (const float*)k, (const float*)v, len, (int32_t)H, (int32_t)KVH,
                               (int32_t)D, scale, per, ws);
        if (nb > 1)
            hipLaunchKernelGGL(k_attention_combine<float>, dim3((unsigned)H), dim3(combine_threads(nb, D)), 0, s, (float*)out, ws,
                               (int32_t)nb, (int32_t)H, (int32_t)D);
    }
    return (int)hipGetLastError();
}

int attention_lds_bytes(int64_t max_len) { return (int)(max_len * 4 > 256 * 4 ? max_len * 4 : 256 * 4); }
// longest attention span served: its scores plus the kernel's static LDS stay
// within 64 KB
int64_t attention_max_len() { return 16000; }

int launch_attention(void* out, const void* q, const void* k, const void* v, int64_t n_q, int64_t len0, int64_t H,
                     int64_t KVH, int64_t D, float scale, int dtype, void* stream)
{
    const dim3 grid((unsigned)H, (unsigned)n_q);
    const size_t lds = (size_t)attention_lds_bytes(len0 + n_q - 1);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16)
        hipLaunchKernelGGL(k_attention<f16>, grid, dim3(256), lds, s, (f16*)out, (const f16*)q, (const f16*)k,
                           (const f16*)v, len0, H, KVH, D, scale);
    else
        hipLaunchKernelGGL(k_attention<float>, grid, dim3(256), lds, s, (float*)out, (const float*)q, (const float*)k,
                           (const float*)v, len0, H, KVH, D, scale);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dense linear with fp32 or fp16 weights W [N, K] (the fp32 model path and
// the tied LM head): out[m][n] = sum_k x[m][k] W[n][k] + bias[n] (+ res[m][n]).
// One wave per output row n and up to 4 activation rows per pass; lanes
// stride K with 16-byte weight loads when K is a multiple of the vector
// width, then a butterfly sum.  Memory-bound: the weights are read once per
// 4 rows of M.
// ---------------------------------------------------------------------------
template <typename T, typename WT>
__global__ __launch_bounds__(256) void k_dense(T* __restrict__ out, const T* __restrict__ x, const WT* __restrict__ w,
                                               const float* __restrict__ bias, const T* res, int64_t M, int64_t N,
                                               int64_t K)
{
    const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n >= N) return;
    const WT* wr = w + n * K;
    for (int64_t m0 = 0; m0 < M; m0 += 4) {
        const int mr = (int)(M - m0 < 4 ? M - m0 : 4);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int64_t kk = lane; kk < K; kk += 64) {
            const float wv = (float)wr[kk];
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (r < mr) acc[r] += ldf(x, (m0 + r) * K + kk) * wv;
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float a = acc[r];
            for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off);
            acc[r] = a;
        }
        if (lane == 0) {
            for (int r = 0; r < mr; r++) {
                const int64_t o = (m0 + r) * N + n;
                float y = acc[r] + (bias ? bias[n] : 0.0f);
                if (res) y += ldf(res, o);
                stf(out, o, y);
            }
        }
    }
}

// Same product with 16-byte loads (K a multiple of 8, x and w 16-byte
// aligned): lane l takes elements [8 l, 8 l + 8) of each 512-wide k step,
// four steps' weight loads in flight before their FMAs.
template <typename T, typename WT>
__global__ __launch_bounds__(256) void k_dense_vec(T* __restrict__ out, const T* __restrict__ x,
                                                   const WT* __restrict__ w, const float* __restrict__ bias,
                                                   const T* res, int64_t M, int64_t N, int64_t K)
{
    const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n >= N) return;
    const WT* wr = w + n * K;
    for (int64_t m0 = 0; m0 < M; m0 += 4) {
        const int mr = (int)(M - m0 < 4 ? M - m0 : 4);
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int64_t k0 = (int64_t)lane * 8; k0 < K; k0 += 4 * 512) {
            float wf[4][8];
#pragma unroll
            for (int u = 0; u < 4; u++)
                if (k0 + u * 512 < K) load8(wr + k0 + u * 512, wf[u]);
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (k0 + u * 512 < K) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        if (r < mr) {
                            float xf[8];
                            load8(x + (m0 + r) * K + k0 + u * 512, xf);
#pragma unroll
                            for (int e = 0; e < 8; e++) acc[r] += xf[e] * wf[u][e];
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float a = acc[r];
            for (int off = 32; off > 0; off >>= 1) a += __shfl_xor(a, off);
            acc[r] = a;
        }
        if (lane == 0) {
            for (int r = 0; r < mr; r++) {
                const int64_t o = (m0 + r) * N + n;
                float y = acc[r] + (bias ? bias[n] : 0.0f);
                if (res) y += ldf(res, o);
                stf(out, o, y);
            }
        }
    }
}

// The same product for M <= 4 activation rows over many weight rows (the
// tied LM head, 151936 x 896 fp16 weights), laid out like the int8 decode
// kernel k_dot: a wave owns a tile of 16 weight rows, lane l reads the
// 16-byte chunk l % 8 of one 128-byte line of rows n0 + l / 8 and
// n0 + 8 + l / 8, so every load instruction covers 8 rows x one whole cache
// line, and a ring of D k steps (one line of each row per step) is in flight;
// each slot also carries the lane's activation chunk of that step.  While
// steps remain beyond the ring, the slot consumed is refilled with the step D
// ahead (past the range it re-reads the last step, never consumed), so every
// wait counts the same D - 1 steps of loads.  fp16 x fp16 products go
// through v_dot2_f32_f16 (exact products, fp32 sums), other types through
// fp32 FMAs; the 8 chunk lanes of a row are summed at the end.  k_dense_vec
// keeps one row per wave and two 16-byte loads in flight per lane, which
// held the LM head to 4.1 TB/s.
template <typename T, int E>
struct alignas(sizeof(T) * E >= 16 ? 16 : sizeof(T) * E) DenseX {
    T v[E];
};

template <typename T, typename WT, int MT, int D>
__global__ __launch_bounds__(256) void k_dense_stream(T* __restrict__ out, const T* __restrict__ x,
                                                      const WT* __restrict__ w, const float* __restrict__ bias,
                                                      const T* res, int64_t M, int64_t N, int64_t K)
{
    constexpr int E = 16 / (int)sizeof(WT);  // weights per 16-byte chunk
    constexpr int STEP = 8 * E;              // k per step: one 128-byte line of each row
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane >> 3, c = lane & 7;
    const int64_t n0 = ((int64_t)blockIdx.x * 4 + wave) * 16;
    if (n0 >= N) return;  // no block-wide synchronisation below
    const int64_t rowA = n0 + r < N ? n0 + r : N - 1;
    const int64_t rowB = n0 + 8 + r < N ? n0 + 8 + r : N - 1;
    const WT* wa = w + rowA * K;
    const WT* wb = w + rowB * K;
    const int32_t steps = (int32_t)((K + STEP - 1) / STEP);
    const int32_t kmax = (int32_t)K - E;  // last chunk start of a row (K % E == 0)
    struct Slot {
        u4 wA, wB;
        DenseX<T, E> xv[MT];
    };
    Slot ring[D];
    auto issue = [&](int u, int32_t st) {
        st = st < steps ? st : steps - 1;  // past the range: re-read the last step (never consumed)
        int32_t k = st * STEP + c * E;
        k = k < kmax ? k : kmax;
        ring[u].wA = __builtin_nontemporal_load(reinterpret_cast<const u4*>(wa + k));
        ring[u].wB = __builtin_nontemporal_load(reinterpret_cast<const u4*>(wb + k));
#pragma unroll
        for (int m = 0; m < MT; m++)
            ring[u].xv[m] = *reinterpret_cast<const DenseX<T, E>*>(x + (m < M ? m : 0) * K + k);
    };
    float accA[MT], accB[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) accA[m] = accB[m] = 0.0f;
    auto consume = [&](int u, int32_t st) {
        const bool kv = st * STEP + c * E < K;  // chunk inside the row (a K tail reads a clamped chunk)
        if constexpr (sizeof(WT) == 2 && sizeof(T) == 2) {
            const h8 a = __builtin_bit_cast(h8, ring[u].wA), b = __builtin_bit_cast(h8, ring[u].wB);
#pragma unroll
            for (int m = 0; m < MT; m++) {
                h8 xh = __builtin_bit_cast(h8, ring[u].xv[m]);
                xh = (kv && m < M) ? xh : h8{};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    accA[m] = __builtin_amdgcn_fdot2(h2{a[2 * j], a[2 * j + 1]}, h2{xh[2 * j], xh[2 * j + 1]},
                                                     accA[m], false);
                    accB[m] = __builtin_amdgcn_fdot2(h2{b[2 * j], b[2 * j + 1]}, h2{xh[2 * j], xh[2 * j + 1]},
                                                     accB[m], false);
                }
            }
        } else {
            const auto a = __builtin_bit_cast(DenseX<WT, E>, ring[u].wA);
            const auto b = __builtin_bit_cast(DenseX<WT, E>, ring[u].wB);
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const bool on = kv && m < M;
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const float xf = on ? (float)ring[u].xv[m].v[e] : 0.0f;
                    accA[m] += xf * (float)a.v[e];
                    accB[m] += xf * (float)b.v[e];
                }
            }
        }
    };
    int32_t st = 0;
#pragma unroll
    for (int u = 0; u < D; u++) issue(u, u);
    for (; st + D < steps; st += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            consume(u, st + u);
            __builtin_amdgcn_sched_barrier(0);
            issue(u, st + u + D);
        }
    }
#pragma unroll
    for (int u = 0; u < D; u++)
        if (st + u < steps) consume(u, st + u);
#pragma unroll
    for (int m = 0; m < MT; m++) {
        accA[m] = group_sum(accA[m], 8);
        accB[m] = group_sum(accB[m], 8);
    }
    if (c != 0) return;
#pragma unroll
    for (int m = 0; m < MT; m++) {
        if (m >= M) continue;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int64_t n = n0 + 8 * h + r;
            if (n >= N) continue;
            const int64_t o = m * N + n;
            float y = (h ? accB[m] : accA[m]) + (bias ? bias[n] : 0.0f);
            if (res) y += ldf(res, o);
            stf(out, o, y);
        }
    }
}

// rows of weights from which the streaming form pays (one block of 4 wave
// tiles of 16 rows per CU at least)
constexpr int64_t kDenseStreamMinN = 16384;

template <typename T, typename WT>
static void dense_stream_go(void* out, const void* x, const void* w, const float* bias, const void* res, int64_t M,
                            int64_t N, int64_t K, hipStream_t s)
{
    constexpr int E = 16 / (int)sizeof(WT);
    const int64_t steps = (K + 8 * E - 1) / (8 * E);
    const dim3 grid((unsigned)(((N + 15) / 16 + 3) / 4));
#define VVH_DS(MT, D)                                                                                                     hipLaunchKernelGGL((k_dense_stream<T, WT, MT, D>), grid, dim3(256), 0, s, (T*)out, (const T*)x, (const WT*)w,                          bias, (const T*)res, M, N, K)
    if (M == 1) {
        if (steps >= 7) VVH_DS(1, 7);
        else VVH_DS(1, 4);
    } else if (M == 2) {
        if (steps >= 7) VVH_DS(2, 7);
        else VVH_DS(2, 4);
    } else {
        VVH_DS(4, 4);
    }
#undef VVH_DS
}

int launch_dense(void* out, const void* x, const void* w, int wdtype, const float* bias, const void* res, int64_t M,
                 int64_t N, int64_t K, int dtype, void* stream)
{
    const dim3 grid((unsigned)((N + 3) / 4));
    hipStream_t s = static_cast<hipStream_t>(stream);
    {
        // the streaming form: M <= 4, many rows, rows of whole 16-byte chunks,
        // 16-byte aligned weights and activations aligned for their chunks
        const int64_t e = wdtype == VVH_F16 ? 8 : 4;
        const uintptr_t xal = (uintptr_t)(e * (dtype == VVH_F16 ? 2 : 4));
        const bool stream_ok = M >= 1 && M <= 4 && N >= kDenseStreamMinN && K >= e && K % e == 0 &&
                               reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                               reinterpret_cast<uintptr_t>(x) % (xal < 16 ? xal : 16) == 0;
        if (stream_ok) {
            if (dtype == VVH_F16) {
                if (wdtype == VVH_F16) dense_stream_go<f16, f16>(out, x, w, bias, res, M, N, K, s);
                else dense_stream_go<f16, float>(out, x, w, bias, res, M, N, K, s);
            } else {
                if (wdtype == VVH_F16) dense_stream_go<float, f16>(out, x, w, bias, res, M, N, K, s);
                else dense_stream_go<float, float>(out, x, w, bias, res, M, N, K, s);
            }
            return (int)hipGetLastError();
        }
    }
    const bool vec = K % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
#define VVH_DENSE(T, WT)                                                                                              \
    if (vec)                                                                                                          \
        hipLaunchKernelGGL((k_dense_vec<T, WT>), grid, dim3(256), 0, s, (T*)out, (const T*)x, (const WT*)w, bias,   \
                           (const T*)res, M, N, K);                                                                   \
    else                                                                                                              \
        hipLaunchKernelGGL((k_dense<T, WT>), grid, dim3(256), 0, s, (T*)out, (const T*)x, (const WT*)w, bias,       \
                           (const T*)res, M, N, K);
    if (dtype == VVH_F16) {
        if (wdtype == VVH_F16) {
            VVH_DENSE(f16, f16)
        } else {
            VVH_DENSE(f16, float)
        }
    } else {
        if (wdtype == VVH_F16) {
            VVH_DENSE(float, f16)
        } else {
            VVH_DENSE(float, float)
        }
    }
#undef VVH_DENSE
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// matmul: out[M][N] = A[M][K] @ B[K][N] (B row-major [K, N], fp32).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_matmul(T* __restrict__ out, const T* __restrict__ A, const float* __restrict__ B,
                                                int64_t M, int64_t N, int64_t K)
{
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < M * N; o += (int64_t)gridDim.x * 256) {
        const int64_t i = o / N, j = o - (o / N) * N;
        float sum = 0.0f;
        for (int64_t kk = 0; kk < K; kk++) sum += ldf(A, i * K + kk) * B[kk * N + j];
        stf(out, o, sum);
    }
}

int launch_matmul(void* out, const void* A, const float* B, int64_t M, int64_t N, int64_t K, int dtype, void* stream)
{
    const int64_t want = (M * N + 255) / 256;
    const dim3 grid((unsigned)(want < 8192 ? (want > 0 ? want : 1) : 8192));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16) hipLaunchKernelGGL(k_matmul<f16>, grid, dim3(256), 0, s, (f16*)out, (const f16*)A, B, M, N, K);
    else hipLaunchKernelGGL(k_matmul<float>, grid, dim3(256), 0, s, (float*)out, (const float*)A, B, M, N, K);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// Sampling over n logits (fp32, or fp16 widened exactly).
//
// Greedy (argmax): the first index of the maximum, as std::max_element
// (src/sampler/sampler.cc:21-25).
//
// Gumbel-max (temperature > 0), the device sampler of the reference
// (src/backend/cuda_kernels.cu:1240-1317 via cuda_sample :1322-1349): index
// argmax_i of logit_i / T + g_i with g_i = -log(-log(u_i)) and u_i the hash
// uniform of (seed, step, i) (:1228-1237).  As there, a candidate counts
// only when its noisy value is > -1e30 (NaN never counts) and the index is 0
// when none does.  Equal noisy values resolve to the lower index (the
// reference's single block keeps the lower thread's, a measure-zero event).
//
// Block b takes the span [b * per, (b + 1) * per) and writes its (best
// value, index) to the workspace; one block then merges the partials in block
// order.  A single block writes the index directly.
// ---------------------------------------------------------------------------
// (v, i) = the better of (v, i) and (ov, oi): larger value, then lower index
__device__ __forceinline__ void argmax_merge(float& v, int64_t& i, float ov, int64_t oi)
{
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

__device__ __forceinline__ void argmax_block(float& best, int64_t& besti)
{
    __shared__ float bv[4];
    __shared__ int64_t bi[4];
    for (int off = 32; off > 0; off >>= 1) argmax_merge(best, besti, __shfl_xor(best, off), __shfl_xor(besti, off));
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = besti;
    }
    __syncthreads();
    best = bv[0];
    besti = bi[0];
    for (int w = 1; w < 4; w++) argmax_merge(best, besti, bv[w], bi[w]);
}

// The reference's hash uniform in (0, 1] (cuda_kernels.cu:1228-1237): the
// seed xor a Weyl sequence of step and index, through the splitmix64
// finaliser, top 53 bits scaled to [0, 1) in fp32, plus 1e-10.
__device__ __forceinline__ float sample_uniform(uint64_t seed, int32_t step, int32_t idx)
{
    uint64_t h = seed ^ ((uint64_t)(int64_t)step * 0x9E3779B97F4A7C15ull + (uint64_t)(int64_t)idx * 0x517CC1B727220A95ull);
    h = (h ^ (h >> 30)) * 0xBF58476D1CE4E5B9ull;
    h = (h ^ (h >> 27)) * 0x94D049BB133111EBull;
    h ^= h >> 31;
    return (float)(h >> 11) * (1.0f / 9007199254740992.0f) + 1e-10f;
}

constexpr int64_t kNone = INT64_MAX;  // partial of a block in which no candidate counted

template <typename T, bool GUMBEL>
__global__ __launch_bounds__(256) void k_sample_part(const T* __restrict__ x, int64_t n, int64_t per, float temperature,
                                                     uint64_t seed, int32_t step, float* __restrict__ pv,
                                                     int64_t* __restrict__ pi, int32_t* __restrict__ idx)
{
    const int64_t b0 = (int64_t)blockIdx.x * per;
    const int64_t e = b0 + per < n ? b0 + per : n;
    float best = GUMBEL ? -1e30f : -INFINITY;
    int64_t besti = kNone;
    for (int64_t i = b0 + threadIdx.x; i < e; i += 256) {  // increasing i: strictly greater keeps the first
        float v = (float)x[i];
        if (GUMBEL) {
            const float u = sample_uniform(seed, step, (int32_t)i);
            v = v / temperature + -logf(-logf(u));
            if (v > best) {
                best = v;
                besti = i;
            }
        } else if (besti == kNone || v > best) {  // the span is never empty: every block has a first element
            best = v;
            besti = i;
        }
    }
    argmax_block(best, besti);
    if (threadIdx.x == 0) {
        if (gridDim.x == 1) {
            idx[0] = (int32_t)(besti == kNone ? 0 : besti);
        } else {
            pv[blockIdx.x] = best;
            pi[blockIdx.x] = besti;
        }
    }
}

__global__ __launch_bounds__(256) void k_sample_final(const float* __restrict__ pv, const int64_t* __restrict__ pi,
                                                      int32_t nb, int32_t* __restrict__ idx)
{
    float best = -INFINITY;
    int64_t besti = kNone;
    for (int b = threadIdx.x; b < nb; b += 256) argmax_merge(best, besti, pv[b], pi[b]);
    argmax_block(best, besti);
    if (threadIdx.x == 0) idx[0] = (int32_t)(besti == kNone ? 0 : besti);
}

constexpr int64_t kArgmaxPer = 2048;  // elements per block
constexpr int64_t kArgmaxMaxBlocks = 1024;

int64_t argmax_ws_bytes(int64_t n)
{
    const int64_t per = std::max(kArgmaxPer, (n + kArgmaxMaxBlocks - 1) / kArgmaxMaxBlocks);
    const int64_t nb = (n + per - 1) / per;
    return nb > 1 ? nb * 12 : 0;
}

int launch_sample(const void* x, int dtype, int64_t n, float temperature, uint64_t seed, int32_t step, int32_t* idx,
                  float* ws, void* stream)
{
    const int64_t per = std::max(kArgmaxPer, (n + kArgmaxMaxBlocks - 1) / kArgmaxMaxBlocks);
    const int64_t nb = (n + per - 1) / per;
    hipStream_t s = static_cast<hipStream_t>(stream);
    int64_t* pi = reinterpret_cast<int64_t*>(ws);  // nb int64 indices, then nb fp32 values
    float* pv = ws ? reinterpret_cast<float*>(pi + nb) : nullptr;
    const dim3 grid((unsigned)nb);
    const bool g = temperature != 0.0f;
    if (dtype == VVH_F16) {
        if (g) hipLaunchKernelGGL((k_sample_part<f16, true>), grid, dim3(256), 0, s, (const f16*)x, n, per, temperature, seed, step, pv, pi, idx);
        else hipLaunchKernelGGL((k_sample_part<f16, false>), grid, dim3(256), 0, s, (const f16*)x, n, per, temperature, seed, step, pv, pi, idx);
    } else {
        if (g) hipLaunchKernelGGL((k_sample_part<float, true>), grid, dim3(256), 0, s, (const float*)x, n, per, temperature, seed, step, pv, pi, idx);
        else hipLaunchKernelGGL((k_sample_part<float, false>), grid, dim3(256), 0, s, (const float*)x, n, per, temperature, seed, step, pv, pi, idx);
    }
    if (nb > 1) hipLaunchKernelGGL(k_sample_final, dim3(1), dim3(256), 0, s, pv, pi, (int32_t)nb, idx);
    return (int)hipGetLastError();
}

int launch_argmax(const float* x, int64_t n, int32_t* idx, float* ws, void* stream)
{
    return launch_sample(x, VVH_F32, n, 0.0f, 0, 0, idx, ws, stream);
}

}  // namespace vvh
