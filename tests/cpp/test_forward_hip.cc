// Whole forward passes of a small Qwen2-shaped model through the vvllm
// Backend and KVCache interfaces only, in the operator order of the
// reference's transformer_forward (include/vvllm/model/transformer.h:76-215,
// with linear / linear_add / rms_norm_seq of src/model/transformer.cc:6-50):
// embedding (fp32, converted in fp16 mode), per layer rms_norm per token,
// q/k/v linear_q8 with bias, rope, KV append, causal_attention per query,
// o linear_q8_add in place, rms_norm, gate_up linear_q8, silu_mul per token,
// down linear_q8_add in place; then the final rms_norm of the last token and
// the tied-embedding LM head (dense linear), logits in fp32.
//
// The same forward runs on BackendHIP + KVCacheHIP (device activations) and
// on a CPU Backend built from the oracle's restatement of BackendCPU (test
// infrastructure: oracle/oracle.c), for a 20-token prompt (the GEMM paths,
// M = 20, and K = 96, not a multiple of 64) and 6 decode steps (M = 1).
// With fp16 activations the CPU backend stores every operator's output as
// fp16, as the device does (fp32 arithmetic inside each operator, the dense
// LM head's weights in fp16), so both sides round at the same places.
//
// Every operator's output is recorded on both sides; each step's logits must
// agree within a normalized max error of 1e-4 (fp32) or 1e-2 (fp16), with
// the same greedy token.  On a failure the per-operator errors of that step
// are printed, naming the first operator that diverges.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "backend_hip.h"
#include "half.h"
#include "oracle.h"
#include "vvllm/backend/backend.h"
#include "vvllm/kv_cache/kv_cache.h"

namespace
{

using vvllm::Backend;
using vvllm::KVCache;

struct Cfg {
    std::size_t hidden = 64, heads = 4, kv_heads = 2, head_dim = 16, inter = 96, layers = 2, vocab = 128;
    float eps = 1e-6f, theta = 10000.0f;
    std::size_t kv_dim() const { return kv_heads * head_dim; }
};

struct Q8 {
    std::vector<int8_t> q;
    std::vector<float> s;
};

struct Layer {
    std::vector<float> ln1, ln2, qb, kb, vb;
    Q8 q, k, v, o, gu, down;
};

struct Model {
    Cfg c;
    std::vector<float> table, final_norm;
    std::vector<Layer> layers;
};

struct Rng {
    std::uint64_t s;
    float normal()
    {
        // sum of 12 uniforms - 6: an approximately N(0, 1), deterministic draw
        float acc = 0;
        for (int i = 0; i < 12; i++) {
            s = s * 6364136223846793005ull + 1442695040888963407ull;
            acc += (float)((s >> 40) & 0xFFFFFF) / 16777216.0f;
        }
        return acc - 6.0f;
    }
};

Q8 quantized(Rng& r, std::size_t N, std::size_t K, float std)
{
    std::vector<float> w(N * K);
    for (auto& v : w) v = std * r.normal();
    Q8 out;
    out.q.resize(N * K);
    out.s.resize(N);
    orc_quantize_per_channel(w.data(), N, K, out.q.data(), out.s.data());
    return out;
}

std::vector<float> vec(Rng& r, std::size_t n, float mean, float std)
{
    std::vector<float> v(n);
    for (auto& x : v) x = mean + std * r.normal();
    return v;
}

Model make_model(std::uint64_t seed)
{
    Model m;
    Rng r{seed};
    const Cfg& c = m.c;
    m.table = vec(r, c.vocab * c.hidden, 0.0f, 0.5f);
    m.final_norm = vec(r, c.hidden, 1.0f, 0.1f);
    for (std::size_t l = 0; l < c.layers; l++) {
        Layer L;
        L.ln1 = vec(r, c.hidden, 1.0f, 0.1f);
        L.ln2 = vec(r, c.hidden, 1.0f, 0.1f);
        L.q = quantized(r, c.heads * c.head_dim, c.hidden, 0.1f);
        L.k = quantized(r, c.kv_dim(), c.hidden, 0.1f);
        L.v = quantized(r, c.kv_dim(), c.hidden, 0.1f);
        L.qb = vec(r, c.heads * c.head_dim, 0.0f, 0.1f);
        L.kb = vec(r, c.kv_dim(), 0.0f, 0.1f);
        L.vb = vec(r, c.kv_dim(), 0.0f, 0.1f);
        L.o = quantized(r, c.hidden, c.heads * c.head_dim, 0.1f);
        L.gu = quantized(r, 2 * c.inter, c.hidden, 0.1f);
        L.down = quantized(r, c.hidden, c.inter, 0.1f);
        m.layers.push_back(std::move(L));
    }
    return m;
}

// Activation storage of one side: fp32, or fp16 bits behind the float*.
struct Store {
    bool fp16;
    std::size_t elem() const { return fp16 ? 2 : 4; }
    std::vector<float> load(const void* p, std::size_t n) const
    {
        std::vector<float> v(n);
        if (fp16) {
            const auto* h = static_cast<const std::uint16_t*>(p);
            for (std::size_t i = 0; i < n; i++) v[i] = from_half(h[i]);
        } else {
            std::memcpy(v.data(), p, n * 4);
        }
        return v;
    }
    void store(void* p, const float* v, std::size_t n) const
    {
        if (fp16) {
            auto* h = static_cast<std::uint16_t*>(p);
            for (std::size_t i = 0; i < n; i++) h[i] = to_half(v[i]);
        } else {
            std::memcpy(p, v, n * 4);
        }
    }
    void store(void* p, const std::vector<float>& v) const { store(p, v.data(), v.size()); }
};

// ---- the CPU side: the oracle's BackendCPU restatement behind the interface.
// Each operator widens its activation inputs, runs the oracle in fp32 and
// stores its output in the activation dtype.
class OracleBackend : public Backend
{
public:
    explicit OracleBackend(bool fp16) : st_{fp16} {}

    void* allocate(std::size_t bytes) override { return std::malloc(bytes); }
    void deallocate(void* p) override { std::free(p); }
    bool is_fp16() const override { return st_.fp16; }
    void fp32_to_fp16(void* dst, const float* src, std::size_t n) override { Store{true}.store(dst, src, n); }
    void fp16_to_fp32(float* dst, const void* src, std::size_t n) override
    {
        const auto v = Store{true}.load(src, n);
        std::memcpy(dst, v.data(), n * 4);
    }

    void matmul(float* o, const float* A, const float* B, std::size_t M, std::size_t N, std::size_t K) override
    {
        const auto a = ld(A, M * K);
        std::vector<float> r(M * N);
        orc_matmul(r.data(), a.data(), B, M, N, K);
        st_.store(o, r);
    }
    void add(float* o, const float* x, const float* y, std::size_t n) override { binary(orc_add, o, x, y, n); }
    void mul(float* o, const float* x, const float* y, std::size_t n) override { binary(orc_mul, o, x, y, n); }
    void silu_mul(float* o, const float* g, const float* u, std::size_t n) override
    {
        binary(orc_silu_mul, o, g, u, n);
    }
    void silu(float* o, const float* x, std::size_t n) override
    {
        const auto a = ld(x, n);
        std::vector<float> r(n);
        orc_silu(r.data(), a.data(), n);
        st_.store(o, r);
    }
    void softmax(float* o, const float* x, std::size_t n) override
    {
        const auto a = ld(x, n);
        std::vector<float> r(n);
        orc_softmax(r.data(), a.data(), n);
        st_.store(o, r);
    }
    void rms_norm(float* o, const float* x, const float* w, std::size_t n, float eps) override
    {
        const auto a = ld(x, n);
        std::vector<float> r(n);
        orc_rms_norm(r.data(), a.data(), w, n, eps);
        st_.store(o, r);
    }
    void rope(float* q, float* k, std::size_t S, std::size_t H, std::size_t KVH, std::size_t D, std::size_t pos,
              float theta) override
    {
        auto a = ld(q, S * H * D), b = ld(k, S * KVH * D);
        orc_rope(a.data(), b.data(), S, H, KVH, D, pos, theta);
        st_.store(q, a);
        st_.store(k, b);
    }
    // the device mirrors a dense weight in the activation dtype
    void linear(float* o, const float* x, const float* w, const float* b, std::size_t M, std::size_t N,
                std::size_t K) override
    {
        linear_add(o, x, w, b, nullptr, M, N, K);
    }
    void linear_add(float* o, const float* x, const float* w, const float* b, const float* res, std::size_t M,
                    std::size_t N, std::size_t K) override
    {
        const auto a = ld(x, M * K);
        std::vector<float> wr(w, w + N * K);
        if (st_.fp16)
            for (auto& v : wr) v = from_half(to_half(v));
        std::vector<float> r(M * N);
        if (res) {
            const auto rr = ld(res, M * N);
            orc_linear_add(r.data(), a.data(), wr.data(), b, rr.data(), M, N, K);
        } else {
            orc_linear(r.data(), a.data(), wr.data(), b, M, N, K);
        }
        st_.store(o, r);
    }
    void linear_q8(float* o, const float* x, const int8_t* w, const float* s, const float* b, std::size_t M,
                   std::size_t N, std::size_t K) override
    {
        linear_q8_add(o, x, w, s, b, nullptr, M, N, K);
    }
    void linear_q8_add(float* o, const float* x, const int8_t* w, const float* s, const float* b, const float* res,
                       std::size_t M, std::size_t N, std::size_t K) override
    {
        const auto a = ld(x, M * K);
        std::vector<float> r(M * N);
        if (res) {
            const auto rr = ld(res, M * N);
            orc_linear_q8_add(r.data(), a.data(), w, s, b, rr.data(), M, N, K);
        } else {
            orc_linear_q8(r.data(), a.data(), w, s, b, M, N, K);
        }
        st_.store(o, r);
    }
    // BackendCPU::embedding (src/backend/backend_naive.cc:338-342): the fp32
    // table row, in fp32 whatever the activation dtype (transformer.h:94-104
    // converts it afterwards)
    void embedding(float* o, const float* table, std::size_t tok, std::size_t hidden, std::size_t) override
    {
        std::memcpy(o, table + tok * hidden, hidden * sizeof(float));
    }
    void causal_attention(float* o, const float* q, std::size_t qi, const float* k, const float* v, std::size_t len,
                          std::size_t H, std::size_t KVH, std::size_t D, float scale) override
    {
        const auto a = ld(q, (qi + 1) * H * D), kk = ld(k, len * KVH * D), vv = ld(v, len * KVH * D);
        std::vector<float> r(H * D);
        orc_causal_attention(r.data(), a.data(), qi, kk.data(), vv.data(), len, H, KVH, D, scale);
        st_.store(o, r);
    }

private:
    std::vector<float> ld(const void* p, std::size_t n) const { return st_.load(p, n); }
    void binary(void (*f)(float*, const float*, const float*, std::size_t), float* o, const float* x,
                const float* y, std::size_t n)
    {
        const auto a = ld(x, n), b = ld(y, n);
        std::vector<float> r(n);
        f(r.data(), a.data(), b.data(), n);
        st_.store(o, r);
    }

    Store st_;
};

// KVCacheCPU's behaviour (src/kv_cache/kv_cache_cpu.cc) with rows in the
// activation dtype.
class HostKVCache : public KVCache
{
public:
    explicit HostKVCache(bool fp16) : elem_(fp16 ? 2 : 4) {}
    void init(std::size_t num_layers, std::size_t kv_dim) override
    {
        if (!k_.empty()) return;
        kv_dim_ = kv_dim;
        k_.resize(num_layers);
        v_.resize(num_layers);
    }
    void append(std::size_t layer, const float* k, const float* v, std::size_t n) override
    {
        const std::size_t row = kv_dim_ * elem_;
        k_[layer].resize((seq_len_ + n) * row);
        v_[layer].resize((seq_len_ + n) * row);
        std::memcpy(k_[layer].data() + seq_len_ * row, k, n * row);
        std::memcpy(v_[layer].data() + seq_len_ * row, v, n * row);
    }
    const float* k(std::size_t layer) const override { return reinterpret_cast<const float*>(k_[layer].data()); }
    const float* v(std::size_t layer) const override { return reinterpret_cast<const float*>(v_[layer].data()); }
    void reset() override { seq_len_ = 0; }
    void truncate(std::size_t n) override
    {
        if (n < seq_len_) seq_len_ = n;
    }

private:
    std::size_t elem_;
    std::vector<std::vector<unsigned char>> k_, v_;  // bytes; vector storage is suitably aligned
};

// Memory of one side's device (the host heap for the CPU backend).
struct Mem {
    bool gpu;
    void* alloc(std::size_t bytes) const { return gpu ? vvllm::hip_device_allocate(bytes) : std::malloc(bytes); }
    void free(void* p) const { gpu ? vvllm::hip_device_deallocate(p) : std::free(p); }
    void to_host(void* dst, const void* src, std::size_t bytes) const
    {
        if (gpu) vvllm::hip_copy_d2h(dst, src, bytes);
        else std::memcpy(dst, src, bytes);
    }
};

using Trace = std::vector<std::pair<std::string, std::vector<float>>>;

// One forward pass of toks at position pos; returns the fp32 logits of the
// last token and appends every operator's output to *trace.
std::vector<float> forward(Backend& be, KVCache& kv, const Mem& mem, const Model& m, const std::vector<int>& toks,
                           std::size_t pos, Trace* trace)
{
    const Cfg& c = m.c;
    const std::size_t S = toks.size(), hidden = c.hidden, H = c.heads, KVH = c.kv_heads, D = c.head_dim;
    const std::size_t kv_dim = c.kv_dim(), I = c.inter;
    const Store st{be.is_fp16()};
    const std::size_t elem = st.elem();
    auto at = [&](void* base, std::size_t i) { return reinterpret_cast<float*>(static_cast<char*>(base) + i * elem); };
    std::vector<void*> owned;
    auto buf = [&](std::size_t elems, std::size_t es) {
        void* p = mem.alloc(elems * es);
        owned.push_back(p);
        return p;
    };
    std::vector<unsigned char> staging;
    auto record = [&](const std::string& name, const void* p, std::size_t n) {
        staging.resize(n * elem);
        mem.to_host(staging.data(), p, n * elem);
        trace->emplace_back(name, st.load(staging.data(), n));
    };

    be.begin_forward();
    kv.init(c.layers, kv_dim);
    if (pos == 0) kv.reset();

    void* x = buf(S * hidden, elem);
    if (be.is_fp16()) {
        void* x32 = buf(S * hidden, 4);
        for (std::size_t s = 0; s < S; s++)
            be.embedding(static_cast<float*>(x32) + s * hidden, m.table.data(), toks[s], hidden, c.vocab);
        be.fp32_to_fp16(x, static_cast<float*>(x32), S * hidden);
    } else {
        for (std::size_t s = 0; s < S; s++) be.embedding(at(x, s * hidden), m.table.data(), toks[s], hidden, c.vocab);
    }
    record("embedding", x, S * hidden);
    void* norm_out = buf(S * hidden, elem);
    void* q = buf(S * H * D, elem);
    void* k_new = buf(S * kv_dim, elem);
    void* v_new = buf(S * kv_dim, elem);
    void* attn_out = buf(S * hidden, elem);
    void* gate_up = buf(S * 2 * I, elem);
    void* gate = buf(S * I, elem);
    const float scale = 1.0f / std::sqrt((float)D);

    for (std::size_t l = 0; l < c.layers; l++) {
        const Layer& L = m.layers[l];
        const std::string p = "layer" + std::to_string(l) + ".";
        for (std::size_t s = 0; s < S; s++)
            be.rms_norm(at(norm_out, s * hidden), at(x, s * hidden), L.ln1.data(), hidden, c.eps);
        record(p + "input_norm", norm_out, S * hidden);
        be.linear_q8(at(q, 0), at(norm_out, 0), L.q.q.data(), L.q.s.data(), L.qb.data(), S, H * D, hidden);
        be.linear_q8(at(k_new, 0), at(norm_out, 0), L.k.q.data(), L.k.s.data(), L.kb.data(), S, kv_dim, hidden);
        be.linear_q8(at(v_new, 0), at(norm_out, 0), L.v.q.data(), L.v.s.data(), L.vb.data(), S, kv_dim, hidden);
        record(p + "q_proj", q, S * H * D);
        record(p + "k_proj", k_new, S * kv_dim);
        record(p + "v_proj", v_new, S * kv_dim);
        be.rope(at(q, 0), at(k_new, 0), S, H, KVH, D, pos, c.theta);
        record(p + "rope.q", q, S * H * D);
        record(p + "rope.k", k_new, S * kv_dim);
        kv.append(l, at(k_new, 0), at(v_new, 0), S);
        for (std::size_t s = 0; s < S; s++)
            be.causal_attention(at(attn_out, s * hidden), at(q, 0), s, kv.k(l), kv.v(l), pos + s + 1, H, KVH, D,
                                scale);
        record(p + "attention", attn_out, S * hidden);
        be.linear_q8_add(at(x, 0), at(attn_out, 0), L.o.q.data(), L.o.s.data(), nullptr, at(x, 0), S, hidden,
                         H * D);
        record(p + "o_proj+residual", x, S * hidden);
        for (std::size_t s = 0; s < S; s++)
            be.rms_norm(at(norm_out, s * hidden), at(x, s * hidden), L.ln2.data(), hidden, c.eps);
        record(p + "post_norm", norm_out, S * hidden);
        be.linear_q8(at(gate_up, 0), at(norm_out, 0), L.gu.q.data(), L.gu.s.data(), nullptr, S, 2 * I, hidden);
        record(p + "gate_up_proj", gate_up, S * 2 * I);
        for (std::size_t s = 0; s < S; s++)
            be.silu_mul(at(gate, s * I), at(gate_up, s * 2 * I), at(gate_up, s * 2 * I + I), I);
        record(p + "silu_mul", gate, S * I);
        be.linear_q8_add(at(x, 0), at(gate, 0), L.down.q.data(), L.down.s.data(), nullptr, at(x, 0), S, hidden, I);
        record(p + "down_proj+residual", x, S * hidden);
    }
    kv.advance(S);

    void* fin = buf(hidden, elem);
    be.rms_norm(at(fin, 0), at(x, (S - 1) * hidden), m.final_norm.data(), hidden, c.eps);
    record("final_norm", fin, hidden);
    void* logits = buf(c.vocab, elem);
    be.linear(at(logits, 0), at(fin, 0), m.table.data(), nullptr, 1, c.vocab, hidden);
    std::vector<float> out(c.vocab);
    if (be.is_fp16()) {
        void* l32 = buf(c.vocab, 4);
        be.fp16_to_fp32(static_cast<float*>(l32), logits, c.vocab);
        mem.to_host(out.data(), l32, c.vocab * 4);
    } else {
        mem.to_host(out.data(), logits, c.vocab * 4);
    }
    trace->emplace_back("logits", out);
    for (void* b : owned) mem.free(b);
    return out;
}

double normalized_error(const std::vector<float>& got, const std::vector<float>& ref)
{
    double mx = 0, err = 0;
    for (std::size_t i = 0; i < ref.size(); i++) {
        mx = std::max(mx, (double)std::fabs(ref[i]));
        const double e = std::fabs((double)got[i] - (double)ref[i]);
        err = std::isnan(e) ? INFINITY : std::max(err, e);
    }
    return err / std::max(mx, 1e-30);
}

int run(bool fp16)
{
    const Model m = make_model(20241201);
    OracleBackend cpu(fp16);
    HostKVCache cpu_kv(fp16);
    vvllm::BackendHIP gpu(fp16);
    vvllm::KVCacheHIP gpu_kv(fp16);
    const Mem cpu_mem{false}, gpu_mem{true};
    const double tol = fp16 ? 1e-2 : 1e-4;
    int failures = 0;

    std::vector<int> toks;
    for (int i = 0; i < 20; i++) toks.push_back((i * 37 + 11) % (int)m.c.vocab);
    std::size_t pos = 0;
    for (int step = 0; step < 7; step++) {
        Trace tr_cpu, tr_gpu;
        const std::vector<float> ref = forward(cpu, cpu_kv, cpu_mem, m, toks, pos, &tr_cpu);
        const std::vector<float> got = forward(gpu, gpu_kv, gpu_mem, m, toks, pos, &tr_gpu);
        const double nerr = normalized_error(got, ref);
        const int tr = (int)(std::max_element(ref.begin(), ref.end()) - ref.begin());
        const int tg = (int)(std::max_element(got.begin(), got.end()) - got.begin());
        std::printf("fp16=%d step %d (pos %zu, %zu tokens): normalized logits error %.2e, next token cpu %d hip %d\n",
                    fp16, step, pos, toks.size(), nerr, tr, tg);
        std::fflush(stdout);
        bool bad = false;
        if (!(nerr <= tol)) {
            std::fprintf(stderr, "  logits error %.3e above %.1e\n", nerr, tol);
            bad = true;
        }
        if (tr != tg) {
            std::fprintf(stderr, "  greedy token differs\n");
            bad = true;
        }
        if (bad) {
            failures++;
            for (std::size_t i = 0; i < tr_cpu.size() && i < tr_gpu.size(); i++)
                std::fprintf(stderr, "    %-28s %.3e\n", tr_cpu[i].first.c_str(),
                             normalized_error(tr_gpu[i].second, tr_cpu[i].second));
        }
        pos += toks.size();
        toks = {tr};  // both sides continue from the CPU's greedy token
    }
    if (gpu_kv.seq_len() != pos) {
        std::fprintf(stderr, "KVCacheHIP length %zu, want %zu\n", gpu_kv.seq_len(), pos);
        failures++;
    }
    return failures;
}

}  // namespace

int main()
{
    int failures = 0;
    for (bool fp16 : {false, true}) {
        std::printf("[case] forward through Backend/KVCache, fp16=%d\n", fp16);
        std::fflush(stdout);
        failures += run(fp16);
    }
    if (failures) {
        std::fprintf(stderr, "test_forward_hip: %d failure(s)\n", failures);
        return 1;
    }
    std::printf("test_forward_hip: all passed\n");
    return 0;
}
