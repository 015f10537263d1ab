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
//   k_argmax     greedy sampling: first index of the max (src/sampler/sampler.cc:21-25)
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
__device__ __forceinline__ float block_sum(float v, float* red)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
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
        else r = (a / (1.0f + expf(-a))) * ldf(y, i);  // silu_mul, backend_naive.cc:297-298
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
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_rms_norm(T* __restrict__ out, const T* __restrict__ x,
                                                  const float* __restrict__ w, int64_t n, float eps)
{
    __shared__ float red[4];
    const T* xr = x + (int64_t)blockIdx.x * n;
    T* orow = out + (int64_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float v = ldf(xr, i);
        ss += v * v;
    }
    ss = block_sum(ss, red);
    const float rms = sqrtf(ss / (float)n + eps);
    for (int64_t i = threadIdx.x; i < n; i += 256) stf(orow, i, ldf(xr, i) / rms * w[i]);
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
template <typename T>
__global__ __launch_bounds__(256) void k_rope(T* __restrict__ q, T* __restrict__ k, int64_t S, int64_t H, int64_t KVH,
                                              int64_t D, int64_t pos, float theta)
{
    const int64_t half = D / 2;
    const int64_t nq = S * H * half, total = nq + S * KVH * half;
    for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < total; g += (int64_t)gridDim.x * 256) {
        T* base;
        int64_t s, i;
        if (g < nq) {
            i = g % half;
            const int64_t hs = g / half;  // s * H + h
            s = hs / H;
            base = q + hs * D;
        } else {
            const int64_t g2 = g - nq;
            i = g2 % half;
            const int64_t hs = g2 / half;
            s = hs / KVH;
            base = k + hs * D;
        }
        const float e = (float)(2 * i) / (float)D;
        const float freq = 1.0f / (float)pow((double)theta, (double)e);
        const float angle = (float)(pos + s) * freq;
        const float c = (float)cos((double)angle), sn = (float)sin((double)angle);
        const float x0 = ldf(base, i), x1 = ldf(base, i + half);
        stf(base, i, x0 * c - x1 * sn);
        stf(base, i + half, x0 * sn + x1 * c);
    }
}

int launch_rope(void* q, void* k, int64_t S, int64_t H, int64_t KVH, int64_t D, int64_t pos, float theta, int dtype,
                void* stream)
{
    const int64_t total = S * (H + KVH) * (D / 2);
    const int64_t want = (total + 255) / 256;
    const dim3 grid((unsigned)(want < 4096 ? (want > 0 ? want : 1) : 4096));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16)
        hipLaunchKernelGGL(k_rope<f16>, grid, dim3(256), 0, s, (f16*)q, (f16*)k, S, H, KVH, D, pos, theta);
    else
        hipLaunchKernelGGL(k_rope<float>, grid, dim3(256), 0, s, (float*)q, (float*)k, S, H, KVH, D, pos, theta);
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

int launch_dense(void* out, const void* x, const void* w, int wdtype, const float* bias, const void* res, int64_t M,
                 int64_t N, int64_t K, int dtype, void* stream)
{
    const dim3 grid((unsigned)((N + 3) / 4));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VVH_F16) {
        if (wdtype == VVH_F16)
            hipLaunchKernelGGL((k_dense<f16, f16>), grid, dim3(256), 0, s, (f16*)out, (const f16*)x, (const f16*)w, bias,
                               (const f16*)res, M, N, K);
        else
            hipLaunchKernelGGL((k_dense<f16, float>), grid, dim3(256), 0, s, (f16*)out, (const f16*)x, (const float*)w,
                               bias, (const f16*)res, M, N, K);
    } else {
        if (wdtype == VVH_F16)
            hipLaunchKernelGGL((k_dense<float, f16>), grid, dim3(256), 0, s, (float*)out, (const float*)x, (const f16*)w,
                               bias, (const float*)res, M, N, K);
        else
            hipLaunchKernelGGL((k_dense<float, float>), grid, dim3(256), 0, s, (float*)out, (const float*)x,
                               (const float*)w, bias, (const float*)res, M, N, K);
    }
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
// argmax over n fp32 values: the first index of the maximum, as
// std::max_element (src/sampler/sampler.cc:21-25).  One block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int64_t n, int32_t* __restrict__ idx)
{
    __shared__ float bv[16];
    __shared__ int64_t bi[16];
    float best = -INFINITY;
    int64_t besti = n;  // n: none seen yet
    for (int64_t i = threadIdx.x; i < n; i += 1024) {  // increasing i: strictly greater keeps the first
        const float v = x[i];
        if (besti == n || v > best) {
            best = v;
            besti = i;
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int64_t oi = __shfl_xor(besti, off);
        if (ov > best || (ov == best && oi < besti)) {
            best = ov;
            besti = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = besti;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int64_t ix = bi[0];
        for (int w = 1; w < 16; w++)
            if (bv[w] > b || (bv[w] == b && bi[w] < ix)) {
                b = bv[w];
                ix = bi[w];
            }
        idx[0] = (int32_t)ix;
    }
}

int launch_argmax(const float* x, int64_t n, int32_t* idx, void* stream)
{
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream), x, n, idx);
    return (int)hipGetLastError();
}

}  // namespace vvh
