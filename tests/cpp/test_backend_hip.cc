// GPU test of BackendHIP through the vvllm Backend interface.
//
// The first cases restate the reference's own tests of the int8 path,
// src/backend/backend_naive_test.cc:355-405 (LinearQ8MatchesFp32) and
// :407-425 (LinearQ8WithBias), run on the MI355X backend in fp32 and in fp16
// mode.  The others cover what the model relies on and the reference never
// tests: linear_q8_add with out == residual (include/vvllm/model/
// transformer.h:165-166), M > 1, the weight mirror refreshing after
// forget_weight, and mirrors released with their backend.
#include <cmath>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "backend_hip.h"
#include "half.h"
#include "vvllm_hip.h"

using vvllm::BackendHIP;
using vvllm::KVCacheHIP;

namespace
{

int g_failures = 0;
#define EXPECT_NEAR(a, b, tol, what)                                                   \
    do {                                                                               \
        const double _a = (a), _b = (b);                                               \
        if (!(std::fabs(_a - _b) <= (tol))) {                                          \
            std::fprintf(stderr, "%s:%d: %s: %.9g vs %.9g (tol %.3g)\n", __FILE__, __LINE__, \
                         what, _a, _b, (double)(tol));                                 \
            g_failures++;                                                              \
        }                                                                              \
    } while (0)

// Activations in the backend's compute dtype, device resident.
struct Act {
    bool fp16;
    std::size_t n;
    void* dev = nullptr;
    Act(bool f, std::size_t count) : fp16(f), n(count) { dev = vvllm::hip_device_allocate(n * (f ? 2 : 4)); }
    ~Act() { vvllm::hip_device_deallocate(dev); }
    void upload(const std::vector<float>& v)
    {
        if (fp16) {
            std::vector<std::uint16_t> h(n);
            for (std::size_t i = 0; i < n; i++) h[i] = to_half(v[i]);
            vvllm::hip_copy_h2d(dev, h.data(), n * 2);
        } else {
            vvllm::hip_copy_h2d(dev, v.data(), n * 4);
        }
    }
    std::vector<float> download()
    {
        std::vector<float> v(n);
        if (fp16) {
            std::vector<std::uint16_t> h(n);
            vvllm::hip_copy_d2h(h.data(), dev, n * 2);
            for (std::size_t i = 0; i < n; i++) v[i] = from_half(h[i]);
        } else {
            vvllm::hip_copy_d2h(v.data(), dev, n * 4);
        }
        return v;
    }
    float* f() { return static_cast<float*>(dev); }
};

// backend_naive_test.cc:355-405, on the HIP backend.
void linear_q8_matches_fp32(bool fp16)
{
    BackendHIP backend(fp16);
    const std::vector<float> weight_fp32 = {0.5f, -0.3f, 0.1f, 0.9f, 1.0f, 0.0f,
                                            -1.0f, 0.5f, 0.0f, 0.2f, 0.4f, -0.8f};
    const std::vector<float> input = {1.0f, 2.0f, 3.0f, 4.0f};
    const std::size_t N = 3, K = 4;
    std::vector<float> out_fp32(N, 0.0f);
    for (std::size_t j = 0; j < N; j++)
        for (std::size_t k = 0; k < K; k++) out_fp32[j] += input[k] * weight_fp32[j * K + k];
    std::vector<int8_t> weight_q8(N * K);
    std::vector<float> scales(N);
    for (std::size_t j = 0; j < N; j++) {
        float absmax = 0.0f;
        for (std::size_t k = 0; k < K; k++) absmax = std::max(absmax, std::fabs(weight_fp32[j * K + k]));
        scales[j] = absmax / 127.0f;
        for (std::size_t k = 0; k < K; k++) {
            float val = weight_fp32[j * K + k] / scales[j];
            val = std::max(-128.0f, std::min(127.0f, std::round(val)));
            weight_q8[j * K + k] = static_cast<int8_t>(val);
        }
    }
    Act in(fp16, K), out(fp16, N);
    in.upload(input);
    backend.linear_q8(out.f(), in.f(), weight_q8.data(), scales.data(), nullptr, 1, N, K);
    const std::vector<float> got = out.download();
    for (std::size_t j = 0; j < N; j++) {
        float tol = scales[j] * static_cast<float>(K) * 0.5f + 1e-5f;
        if (fp16) tol += std::fabs(out_fp32[j]) * 1e-3f;  // fp16 output rounding
        EXPECT_NEAR(got[j], out_fp32[j], tol, fp16 ? "MatchesFp32 fp16" : "MatchesFp32 fp32");
    }
}

// backend_naive_test.cc:407-425, on the HIP backend.
void linear_q8_with_bias(bool fp16)
{
    BackendHIP backend(fp16);
    const std::size_t N = 2, K = 2;
    const std::vector<int8_t> weight = {127, 0, 0, 127};
    const std::vector<float> scales = {1.0f / 127.0f, 1.0f / 127.0f};
    const std::vector<float> bias = {10.0f, 20.0f};
    Act in(fp16, K), out(fp16, N);
    in.upload({3.0f, 5.0f});
    backend.linear_q8(out.f(), in.f(), weight.data(), scales.data(), bias.data(), 1, N, K);
    const std::vector<float> got = out.download();
    const float tol = fp16 ? 1e-2f : 1e-4f;  // 25 in fp16 has an ulp of 1/64
    EXPECT_NEAR(got[0], 13.0f, tol, "WithBias[0]");
    EXPECT_NEAR(got[1], 25.0f, tol, "WithBias[1]");
}

// o_proj / down_proj style call: out == residual, M rows, K a multiple of 64.
void linear_q8_add_inplace(bool fp16, std::size_t M)
{
    BackendHIP backend(fp16);
    const std::size_t N = 96, K = 192;
    std::vector<int8_t> q(N * K);
    std::vector<float> scales(N), bias(N), x(M * K), res(M * N);
    unsigned s = 12345u;
    auto rnd = [&]() { s = s * 1664525u + 1013904223u; return (int)((s >> 8) % 255) - 127; };
    for (auto& v : q) v = (int8_t)rnd();
    for (std::size_t j = 0; j < N; j++) { scales[j] = 0.001f * (1 + j % 7); bias[j] = 0.01f * rnd(); }
    for (auto& v : x) v = 0.05f * rnd();
    for (auto& v : res) v = 0.02f * rnd();
    if (fp16) {  // the device sees fp16 values; use them for the expectation too
        for (auto& v : x) v = from_half(to_half(v));
        for (auto& v : res) v = from_half(to_half(v));
    }
    Act in(fp16, M * K), xo(fp16, M * N);
    in.upload(x);
    xo.upload(res);
    backend.linear_q8_add(xo.f(), in.f(), q.data(), scales.data(), bias.data(), xo.f(), M, N, K);
    const std::vector<float> got = xo.download();
    double maxref = 0, maxerr = 0;
    for (std::size_t i = 0; i < M; i++)
        for (std::size_t j = 0; j < N; j++) {
            double acc = 0;
            for (std::size_t k = 0; k < K; k++) acc += (double)x[i * K + k] * q[j * K + k];
            const double r = acc * scales[j] + bias[j] + res[i * N + j];
            maxref = std::max(maxref, std::fabs(r));
            maxerr = std::max(maxerr, std::fabs(got[i * N + j] - r));
        }
    EXPECT_NEAR(maxerr / maxref, 0.0, fp16 ? 2e-3 : 1e-4, "linear_q8_add in place (normalized)");
}

// A host weight buffer whose contents change after forget_weight is re-mirrored.
void mirror_refresh()
{
    BackendHIP backend(false);
    const std::size_t N = 16, K = 64;
    std::vector<int8_t> q(N * K, 1);
    std::vector<float> scales(N, 1.0f);
    std::vector<float> x(K, 1.0f);
    Act in(false, K), out(false, N);
    in.upload(x);
    backend.linear_q8(out.f(), in.f(), q.data(), scales.data(), nullptr, 1, N, K);
    EXPECT_NEAR(out.download()[0], 64.0, 0.0, "mirror first use");
    std::fill(q.begin(), q.end(), (int8_t)2);
    backend.forget_weight(q.data());
    backend.linear_q8(out.f(), in.f(), q.data(), scales.data(), nullptr, 1, N, K);
    EXPECT_NEAR(out.download()[0], 128.0, 0.0, "mirror after forget_weight");
}

// Mirrors belong to the backend that made them (BackendCUDA frees its weight
// caches in its destructor, backend_cuda.cc:28-35): host buffers rewritten in
// place after their backend is gone are uploaded again by the next backend.
void mirror_per_backend()
{
    const std::size_t N = 16, K = 64;
    std::vector<int8_t> q(N * K, 1);
    std::vector<float> scales(N, 1.0f), norm_w(K, 1.0f);
    std::vector<float> x(K, 1.0f);
    for (int round = 1; round <= 2; round++) {
        BackendHIP backend(false);
        Act in(false, K), out(false, N), normed(false, K);
        in.upload(x);
        backend.linear_q8(out.f(), in.f(), q.data(), scales.data(), nullptr, 1, N, K);
        EXPECT_NEAR(out.download()[0], 64.0 * round, 0.0, "int8 mirror of this backend");
        backend.rms_norm(normed.f(), in.f(), norm_w.data(), K, 1e-6f);
        EXPECT_NEAR(normed.download()[0], 1.0 * round, 1e-5, "norm weight mirror of this backend");
        std::fill(q.begin(), q.end(), (int8_t)2);  // same addresses, new contents
        std::fill(norm_w.begin(), norm_w.end(), 2.0f);
    }
}

// BF16 rows ingested straight into the mirror, then used through linear_q8
// with the rows' address as the weight (what Qwen2Model would pass).
// Row 0 = [1, -1, 0.5, 0, ...]: scale 1/127, codes 127, -127, 64 (63.5 ties
// away from zero), 0; x = e0 + e2 gives 127/127 + 64/127.
void ingest_bf16()
{
    BackendHIP backend(false);
    const std::size_t N = 8, K = 64;
    std::vector<std::uint16_t> rows(N * K, 0);
    auto bf = [](float f) { std::uint32_t u; std::memcpy(&u, &f, 4); return (std::uint16_t)(u >> 16); };
    rows[0] = bf(1.0f); rows[1] = bf(-1.0f); rows[2] = bf(0.5f);
    for (std::size_t j = 1; j < N; j++)
        for (std::size_t k = 0; k < K; k++) rows[j * K + k] = bf(0.01f * (float)((int)((j * 31 + k * 7) % 21) - 10));
    std::vector<float> scales(N), bias(N, 0.5f);
    const int8_t* w = backend.ingest_weight(rows.data(), true, bias.data(), N, K, scales.data());
    EXPECT_NEAR(scales[0], 1.0f / 127.0f, 0.0, "ingested scale");
    std::vector<float> x(K, 0.0f);
    x[0] = 1.0f; x[2] = 1.0f;
    Act in(false, K), out(false, N);
    in.upload(x);
    backend.linear_q8(out.f(), in.f(), w, scales.data(), bias.data(), 1, N, K);
    EXPECT_NEAR(out.download()[0], (127.0 + 64.0) * (1.0f / 127.0f) + 0.5, 1e-5, "ingested row 0");
}

// The other operators through the Backend interface, against double-precision
// restatements of backend_naive.cc, one decode-step's worth of shapes.
void decode_ops(bool fp16)
{
    BackendHIP backend(fp16);
    const std::size_t H = 4, KVH = 2, D = 16, hidden = H * D, vocab = 50;
    unsigned st = 7u;
    auto rnd = [&]() { st = st * 1664525u + 1013904223u; return ((st >> 9) % 2001) / 1000.0f - 1.0f; };
    auto q16 = [&](float v) { return fp16 ? from_half(to_half(v)) : v; };
    double tol = fp16 ? 2e-3 : 1e-4;

    // embedding (always fp32 out) + rms_norm
    std::vector<float> table(vocab * hidden), w(hidden);
    for (auto& v : table) v = rnd();
    for (auto& v : w) v = 1.0f + 0.1f * rnd();
    Act e32(false, hidden), x(fp16, hidden), y(fp16, hidden);
    backend.embedding(e32.f(), table.data(), 17, hidden, vocab);
    std::vector<float> e = e32.download();
    for (std::size_t i = 0; i < hidden; i++) EXPECT_NEAR(e[i], table[17 * hidden + i], 0.0, "embedding");
    std::vector<float> xv(e);
    for (auto& v : xv) v = q16(v);
    x.upload(xv);
    backend.rms_norm(y.f(), x.f(), w.data(), hidden, 1e-6f);
    double ss = 0;
    for (float v : xv) ss += (double)v * v;
    const double rms = std::sqrt(ss / hidden + 1e-6);
    std::vector<float> got = y.download();
    for (std::size_t i = 0; i < hidden; i++) EXPECT_NEAR(got[i], xv[i] / rms * w[i], tol * 3, "rms_norm");

    // silu_mul
    std::vector<float> g(hidden), u(hidden);
    for (std::size_t i = 0; i < hidden; i++) { g[i] = q16(2 * rnd()); u[i] = q16(rnd()); }
    Act dg(fp16, hidden), du(fp16, hidden);
    dg.upload(g);
    du.upload(u);
    backend.silu_mul(y.f(), dg.f(), du.f(), hidden);
    got = y.download();
    for (std::size_t i = 0; i < hidden; i++)
        EXPECT_NEAR(got[i], g[i] / (1.0 + std::exp(-(double)g[i])) * u[i], tol * 2, "silu_mul");

    // rope at position 5 then attention over a KVCacheHIP of 3 positions
    KVCacheHIP cache(fp16);
    cache.init(1, KVH * D);
    std::vector<std::vector<float>> ks, vs;
    for (std::size_t pos = 0; pos < 3; pos++) {
        std::vector<float> qv(H * D), kv(KVH * D), vv(KVH * D);
        for (auto& v : qv) v = q16(rnd());
        for (auto& v : kv) v = q16(rnd());
        for (auto& v : vv) v = q16(rnd());
        Act dq(fp16, H * D), dk(fp16, KVH * D), dv(fp16, KVH * D), out(fp16, H * D);
        dq.upload(qv);
        dk.upload(kv);
        dv.upload(vv);
        backend.rope(dq.f(), dk.f(), 1, H, KVH, D, pos, 10000.0f);
        // expected rotation (split-half pairs)
        auto rot = [&](std::vector<float>& hv, std::size_t heads) {
            for (std::size_t h = 0; h < heads; h++)
                for (std::size_t i = 0; i < D / 2; i++) {
                    const double f = 1.0 / std::pow(10000.0, (double)(2 * i) / D), a = pos * f;
                    const double x0 = hv[h * D + i], x1 = hv[h * D + i + D / 2];
                    hv[h * D + i] = (float)(x0 * std::cos(a) - x1 * std::sin(a));
                    hv[h * D + i + D / 2] = (float)(x0 * std::sin(a) + x1 * std::cos(a));
                }
        };
        rot(qv, H);
        rot(kv, KVH);
        got = dk.download();
        for (std::size_t i = 0; i < KVH * D; i++) EXPECT_NEAR(got[i], kv[i], tol * 4, "rope k");
        ks.push_back(dk.download());
        vs.push_back(vv);
        const std::vector<float> qr = dq.download();
        cache.append(0, dk.f(), dv.f(), 1);
        cache.advance(1);
        const float scale = 1.0f / std::sqrt((float)D);
        backend.causal_attention(out.f(), dq.f(), 0, cache.k(0), cache.v(0), pos + 1, H, KVH, D, scale);
        got = out.download();
        for (std::size_t h = 0; h < H; h++) {
            const std::size_t kh = h / (H / KVH);
            std::vector<double> p(pos + 1);
            double mx = -1e30, sum = 0;
            for (std::size_t t = 0; t <= pos; t++) {
                double dot = 0;
                for (std::size_t d = 0; d < D; d++) dot += (double)qr[h * D + d] * ks[t][kh * D + d];
                p[t] = dot * scale;
                mx = std::max(mx, p[t]);
            }
            for (auto& v : p) { v = std::exp(v - mx); sum += v; }
            for (std::size_t d = 0; d < D; d++) {
                double o = 0;
                for (std::size_t t = 0; t <= pos; t++) o += p[t] / sum * vs[t][kh * D + d];
                EXPECT_NEAR(got[h * D + d], o, tol * 4, "causal_attention over KVCacheHIP");
            }
        }
    }
    if (cache.seq_len() != 3) { std::fprintf(stderr, "kv cache length %zu\n", cache.seq_len()); g_failures++; }

    // dense linear_add (fp32 weights on the host, fp16 on the device in fp16 mode)
    const std::size_t N = 24;
    std::vector<float> W(N * hidden), bias(N), res(N);
    for (auto& v : W) v = 0.1f * rnd();
    for (auto& v : bias) v = rnd();
    for (auto& v : res) v = q16(rnd());
    Act dr(fp16, N);
    dr.upload(res);
    backend.linear_add(dr.f(), x.f(), W.data(), bias.data(), dr.f(), 1, N, hidden);
    got = dr.download();
    for (std::size_t j = 0; j < N; j++) {
        double acc = res[j] + bias[j];
        for (std::size_t k = 0; k < hidden; k++) acc += (double)xv[k] * (fp16 ? from_half(to_half(W[j * hidden + k])) : W[j * hidden + k]);
        EXPECT_NEAR(got[j], acc, tol * 8, "linear_add");
    }
}

}  // namespace

int main()
{
    for (bool fp16 : {false, true}) {
        std::printf("[case] LinearQ8MatchesFp32 fp16=%d\n", fp16); std::fflush(stdout);
        linear_q8_matches_fp32(fp16);
        std::printf("[case] LinearQ8WithBias fp16=%d\n", fp16); std::fflush(stdout);
        linear_q8_with_bias(fp16);
        for (std::size_t M : {1, 5, 40}) {
            std::printf("[case] linear_q8_add in place fp16=%d M=%zu\n", fp16, M); std::fflush(stdout);
            linear_q8_add_inplace(fp16, M);
        }
    }
    std::printf("[case] mirror refresh\n"); std::fflush(stdout);
    mirror_refresh();
    std::printf("[case] mirror per backend\n"); std::fflush(stdout);
    mirror_per_backend();
    std::printf("[case] ingest bf16\n"); std::fflush(stdout);
    ingest_bf16();
    for (bool fp16 : {false, true}) {
        std::printf("[case] decode ops fp16=%d\n", fp16); std::fflush(stdout);
        decode_ops(fp16);
    }
    if (g_failures) {
        std::fprintf(stderr, "test_backend_hip: %d failure(s)\n", g_failures);
        return 1;
    }
    std::printf("test_backend_hip: all passed\n");
    return 0;
}
